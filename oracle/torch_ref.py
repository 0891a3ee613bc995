"""TEST INFRASTRUCTURE ONLY — torch-CPU restatement of the reference's
dequantise-then-matmul path.  Imported only by tests/, smoke() and bench.py's
cpu_baseline leg.

Same op sequence as the reference, on CPU tensors:

* ``dequant``        — ExpertMLPTriton._dequant (kernels/expert_mlp.py:305-330):
                       int8 unpack, interleave, ``int8.to(fp16) * scales``.
* ``expert_mlp``     — ExpertMLPTriton.forward (kernels/expert_mlp.py:292-301):
                       ``silu(x @ Wg.t())``, ``x @ Wu.t()``, product, ``@ Wd.t()``,
                       every tensor fp16 (the MoE fallbacks model/mixtral.py:360-362
                       and model/glm4.py:443-445 are the same F.linear sequence).
* ``mixtral_moe``    — MixtralMoELayer.forward (model/mixtral.py:283-368) with
                       TopKRouter.forward (model/router.py:102-120), affinity off,
                       every expert resident (so unique() ascending order).
* ``glm_moe``        — GLM4MoELayer.forward (model/glm4.py:378-473) with
                       GLM4SigmoidRouter.forward (:279-309); the optional
                       selection bias is this build's extension.

Pins (tests/test_oracle.py), each from outputs the reference's own code wrote
(tests/golden/make_golden.py):
  expert_mlp, dequant           expert_mlp.npz (ExpertMLPTriton.forward), bit for bit
  mixtral_router, mixtral_moe,  mixtral_moe_layer.npz (MixtralMoELayer.forward at
  moe_dispatch                  top-2 and top-1), bit for bit; a per-token brute force
  glm_router, glm_moe,          glm_moe_layer.npz (GLM4MoELayer.forward with its
  dense_mlp                     shared expert), bit for bit; dense_mlp also against
                                float64
  affinity_bonus,               affinity_router.npz (TopKRouter.forward with the
  mixtral_router(cached=...)    cache-affinity bonus), bit for bit
  glm_router with a bias        parity unpinned: the reference has no selection bias;
                                the C oracle's brute-force test covers the selection.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


def dequant(packed: torch.Tensor, scales: torch.Tensor, out_features: int, in_features: int,
            group_size: int) -> torch.Tensor:
    even = (packed & 0x0F).to(torch.int8) - 8
    odd = ((packed >> 4) & 0x0F).to(torch.int8) - 8
    unpacked = torch.zeros(out_features, in_features, dtype=torch.int8, device=packed.device)
    unpacked[:, 0::2] = even
    unpacked[:, 1::2] = odd
    g = unpacked.view(out_features, in_features // group_size, group_size)
    return (g.to(torch.float16) * scales.unsqueeze(-1)).view(out_features, in_features)


def expert_mlp(x, gate_packed, gate_scales, up_packed, up_scales, down_packed, down_scales,
               group_size: int = 128) -> torch.Tensor:
    N = gate_packed.shape[0]
    K = x.shape[-1]
    gate_w = dequant(gate_packed, gate_scales, N, K, group_size)
    up_w = dequant(up_packed, up_scales, N, K, group_size)
    down_w = dequant(down_packed, down_scales, K, N, group_size)
    gate_out = F.silu(x @ gate_w.t())
    up_out = x @ up_w.t()
    return (gate_out * up_out) @ down_w.t()


def mixtral_router(h: torch.Tensor, gate_w: torch.Tensor, top_k: int, cached=None,
                   bonus: float = 0.1, threshold: float = 0.5):
    """logits = fp16 Linear(h).float(); [affinity bonus toward `cached`]; topk;
    softmax; renorm; fp16 (model/router.py:96-120)."""
    logits = F.linear(h, gate_w).float()
    if cached is not None:
        logits = affinity_bonus(logits, cached, bonus, threshold)
    topk_logits, idx = torch.topk(logits, top_k, dim=-1)
    w = F.softmax(topk_logits, dim=-1)
    w = w / w.sum(dim=-1, keepdim=True)
    return idx, w.to(h.dtype), logits


def affinity_bonus(logits: torch.Tensor, cached, bonus: float = 0.1,
                   threshold: float = 0.5) -> torch.Tensor:
    """TopKRouter._apply_affinity_bonus (model/router.py:132-175): + bonus on the
    cached experts' logits of every token whose softmax entropy / ln E exceeds
    the threshold.  cached: iterable of expert ids."""
    E = logits.shape[-1]
    p = F.softmax(logits, dim=-1)
    ent = -(p * torch.log(p + 1e-10)).sum(dim=-1) / math.log(E)
    mask = torch.zeros(E, dtype=logits.dtype)
    for e in cached:
        mask[int(e)] = bonus
    return logits + (ent > threshold).float().unsqueeze(-1) * mask


def glm_router(h: torch.Tensor, w: torch.Tensor, top_k: int, bias=None, eps: float = 1e-9,
               scaling: float = 1.0, n_group: int = 1, topk_group: int = 1,
               norm_topk_prob: bool = True):
    """GLM4SigmoidRouter.forward (model/glm4.py:275-309): fp32 logits, sigmoid,
    group-limited selection when n_group > 1 (group score = max score in the
    group, the topk_group best groups kept, the other experts' scores zeroed,
    :285-298), top-k, weights / (sum + eps) when norm_topk_prob, * scaling, fp16.
    bias (this build's extension): added to the scores for selection only."""
    logits = F.linear(h.float(), w.float())
    scores = torch.sigmoid(logits)
    if n_group > 1 and topk_group > 0:
        E = scores.shape[-1]
        grouped = scores.view(-1, n_group, E // n_group)
        top_groups = grouped.max(dim=-1).values.topk(topk_group, dim=-1).indices
        mask = torch.zeros_like(grouped)
        mask.scatter_(1, top_groups.unsqueeze(-1).expand(-1, -1, E // n_group), 1.0)
        scores = (grouped * mask).view(-1, E)
    if bias is None:
        tw, ti = scores.topk(top_k, dim=-1)
    else:
        _, ti = (scores + bias.float()).topk(top_k, dim=-1)
        tw = scores.gather(-1, ti)
    if norm_topk_prob:
        tw = tw / (tw.sum(dim=-1, keepdim=True) + eps)
    tw = tw * scaling
    return ti, tw.to(h.dtype), logits


def moe_dispatch(flat_hidden, flat_indices, flat_weights, experts, group_size: int = 128):
    """Per-expert gather / expert MLP / fp16 index_add_ (model/mixtral.py:296-368).
    experts: dict e -> (gp, gs, up, us, dp, ds) CPU tensors."""
    unique = flat_indices.unique().tolist()
    out = torch.zeros_like(flat_hidden)
    for e in unique:
        mask = flat_indices == e
        if not mask.any():
            continue
        tok, kpos = torch.where(mask)
        y = expert_mlp(flat_hidden[tok], *experts[e], group_size=group_size)
        out.index_add_(0, tok, y * flat_weights[tok, kpos].unsqueeze(-1))
    return out


def mixtral_moe(h, gate_w, experts, top_k: int = 2, group_size: int = 128, routing=None):
    """h: [T, H] fp16.  routing: optional (idx, w) to reuse a given routing."""
    if routing is None:
        idx, w, _ = mixtral_router(h, gate_w, top_k)
    else:
        idx, w = routing
    return moe_dispatch(h, idx, w, experts, group_size)


def dense_mlp(x, gate_w, up_w, down_w):
    """GLM4DenseMLP.forward (model/glm4.py:234-235), fp16 weights."""
    return F.linear(F.silu(F.linear(x, gate_w)) * F.linear(x, up_w), down_w)


def glm_moe(h, router_w, experts, shared, top_k: int = 8, bias=None, group_size: int = 128,
            routing=None):
    shared_out = dense_mlp(h, *shared)
    if routing is None:
        idx, w, _ = glm_router(h, router_w, top_k, bias=bias)
    else:
        idx, w = routing
    routed = moe_dispatch(h, idx, w, experts, group_size)
    return shared_out + routed

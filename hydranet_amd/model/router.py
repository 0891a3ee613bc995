"""MoE routers on gfx950 (logits GEMV + top-k kernels of libhn_int4.so).

* ``mixtral_route`` / ``TopKRouter`` — model/router.py:73-130: fp16 gate
  Linear with the logits rounded to fp16 and then used as fp32, top-k over the
  logits, softmax over the selected logits, renormalisation, fp16 weights.
  The cache-affinity bonus (model/router.py:132-175) adds a constant to the
  cached experts when the routing entropy is high; when every expert is
  resident it adds the same constant to all logits and changes nothing, so it
  only runs (as three elementwise ops on the logits) if a cache checker
  reports an expert as not resident.
* ``glm_route`` / ``GLM4SigmoidRouter`` — model/glm4.py:238-309: fp32 logits,
  sigmoid, the group-limited selection when n_group > 1 (``group_limit``),
  top-k, weights / (sum + 1e-9) (norm_topk_prob) * routed_scaling_factor, fp16.  An
  optional per-expert bias is added to the scores for selection only (this
  build's extension; the reference loads e_score_correction_bias but does not
  use it, model/glm4_loader.py:164-167).

Ties between equal keys go to the lower expert index (torch's CPU topk leaves
the order of equal values unspecified).  Indices are int32 on the device.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Callable, Optional

import torch
import torch.nn as nn

from .. import _lib


def router_logits(h: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """[T, E] fp32.  fp16 w: logits rounded to fp16 (fp16 Linear); fp32 w: fp32."""
    _lib.require_gpu(h, w)
    T, H = h.shape
    E = w.shape[0]
    hh = _lib.aligned_rows(h.to(torch.float16))
    w_dtype = 0 if w.dtype == torch.float16 else 1
    ww = _lib.aligned_rows(w if w.dtype in (torch.float16, torch.float32) else w.float())
    logits = torch.empty((T, E), dtype=torch.float32, device=h.device)
    _lib.call("hn_router_logits", _lib.ptr(hh), hh.stride(0), _lib.ptr(ww), ww.stride(0), w_dtype,
              _lib.ptr(logits), T, E, H, _lib.stream(h.device))
    return logits


def topk_from_logits(logits: torch.Tensor, k: int, mode: int, bias: Optional[torch.Tensor] = None,
                     eps: float = 1e-9, scaling: float = 1.0):
    """mode 0 = softmax top-k (Mixtral), 1 = sigmoid top-k (GLM).  -> (idx i32, w fp16)."""
    T, E = logits.shape
    lg = logits.contiguous().float()
    b = None if bias is None else bias.to(device=lg.device, dtype=torch.float32).contiguous()
    idx = torch.empty((T, k), dtype=torch.int32, device=lg.device)
    w = torch.empty((T, k), dtype=torch.float16, device=lg.device)
    _lib.call("hn_router_topk", _lib.ptr(lg), _lib.ptr(b), T, E, k, mode, eps, scaling,
              _lib.ptr(idx), _lib.ptr(w), _lib.stream(lg.device))
    return idx, w


def mixtral_route(h: torch.Tensor, gate_w: torch.Tensor, top_k: int = 2):
    """h [T, H] fp16, gate_w [E, H] fp16 -> (idx [T,k] i32, w [T,k] fp16, logits [T,E] f32)."""
    logits = router_logits(h, gate_w)
    idx, w = topk_from_logits(logits, top_k, 0)
    return idx, w, logits


def group_limit(logits: torch.Tensor, n_group: int, topk_group: int) -> torch.Tensor:
    """Group-limited selection (model/glm4.py:285-298): a copy of the [T, E]
    fp32 logits with -inf for the experts outside each token's topk_group
    groups of largest max-sigmoid (sigmoid(-inf) = 0, the reference's masked
    score)."""
    T, E = logits.shape
    lg = logits.contiguous().float()
    out = torch.empty_like(lg)
    _lib.call("hn_router_group_limit", _lib.ptr(lg), T, E, n_group, topk_group, _lib.ptr(out),
              _lib.stream(lg.device))
    return out


def glm_route(h: torch.Tensor, w: torch.Tensor, top_k: int = 8, bias=None, eps: float = 1e-9,
              scaling: float = 1.0, n_group: int = 1, topk_group: int = 1,
              norm_topk_prob: bool = True):
    """GLM4SigmoidRouter.forward's arithmetic: fp32 logits, sigmoid, the
    group-limited selection when n_group > 1 and topk_group > 0, top-k,
    weights / (sum + eps) (norm_topk_prob) * scaling, fp16."""
    logits = router_logits(h, w.float() if w.dtype != torch.float32 else w)
    sel = group_limit(logits, n_group, topk_group) if n_group > 1 and topk_group > 0 else logits
    idx, wt = topk_from_logits(sel, top_k, 1 if norm_topk_prob else 2, bias=bias, eps=eps,
                               scaling=scaling)
    return idx, wt, logits


@dataclass
class RouterOutput:
    expert_indices: torch.Tensor  # (batch, seq, top_k)
    expert_weights: torch.Tensor  # (batch, seq, top_k)
    router_logits: torch.Tensor   # (batch, seq, num_experts)


class TopKRouter(nn.Module):
    """Mixtral top-k router (model/router.py:28-130) on the gfx950 kernels."""

    def __init__(self, hidden_dim: int, num_experts: int, experts_per_token: int = 2,
                 affinity_bonus: float = 0.1, entropy_threshold: float = 0.5,
                 enable_affinity_bonus: bool = False):
        super().__init__()
        self.hidden_dim = hidden_dim
        self.num_experts = num_experts
        self.experts_per_token = experts_per_token
        self.gate = nn.Linear(hidden_dim, num_experts, bias=False)
        self.affinity_bonus = affinity_bonus
        self.entropy_threshold = entropy_threshold
        self.enable_affinity_bonus = enable_affinity_bonus
        self.register_buffer("_one", torch.ones(1, dtype=torch.long), persistent=False)
        self.register_buffer("usage_counts", torch.zeros(num_experts, dtype=torch.long),
                             persistent=False)
        self._is_cached_fn: Optional[Callable[[int], bool]] = None

    def set_cache_checker(self, fn: Callable[[int], bool]):
        self._is_cached_fn = fn

    def _affinity(self, logits: torch.Tensor) -> torch.Tensor:
        if self._is_cached_fn is None:
            return logits
        cached = [bool(self._is_cached_fn(e)) for e in range(self.num_experts)]
        if all(cached) or not any(cached):
            return logits  # a uniform shift changes neither the top-k nor the softmax
        p = torch.softmax(logits, dim=-1)
        ent = -(p * torch.log(p + 1e-10)).sum(-1) / math.log(self.num_experts)
        mask = torch.tensor([self.affinity_bonus if c else 0.0 for c in cached],
                            device=logits.device, dtype=logits.dtype)
        return logits + (ent > self.entropy_threshold).float().unsqueeze(-1) * mask

    def forward(self, hidden_states: torch.Tensor, top_k_override: Optional[int] = None,
                apply_affinity: bool = True) -> RouterOutput:
        B, S, H = hidden_states.shape
        k = top_k_override if top_k_override is not None else self.experts_per_token
        h = hidden_states.reshape(B * S, H)
        logits = router_logits(h, self.gate.weight.to(torch.float16))
        if apply_affinity and self.enable_affinity_bonus:
            logits = self._affinity(logits)
        idx, w = topk_from_logits(logits, k, 0)
        if not self.training:
            # scatter_add_ rather than bincount: no device-to-host sync (graph-capturable)
            flat = idx.view(-1).long()
            self.usage_counts.scatter_add_(0, flat, self._one.expand_as(flat))
        return RouterOutput(idx.view(B, S, k), w.view(B, S, k).to(hidden_states.dtype),
                            logits.view(B, S, self.num_experts))


class GLM4SigmoidRouter(nn.Module):
    """GLM-4.5 sigmoid top-k router (model/glm4.py:238-309) on the gfx950 kernels,
    with group-limited selection (n_group > 1) and norm_topk_prob as the
    reference's."""

    def __init__(self, hidden_dim: int, num_experts: int = 128, top_k: int = 8,
                 norm_topk_prob: bool = True, routed_scaling_factor: float = 1.0,
                 n_group: int = 1, topk_group: int = 1):
        super().__init__()
        if n_group > 1 and topk_group > 0 and num_experts % n_group != 0:
            raise ValueError(f"n_group {n_group} must divide num_experts {num_experts}")
        self.num_experts = num_experts
        self.top_k = top_k
        self.n_group = n_group
        self.topk_group = topk_group
        self.norm_topk_prob = norm_topk_prob
        self.routed_scaling_factor = routed_scaling_factor
        self.weight = nn.Parameter(torch.empty(num_experts, hidden_dim))
        nn.init.kaiming_uniform_(self.weight, a=math.sqrt(5))
        self.register_buffer("selection_bias", None, persistent=False)

    def forward(self, hidden_states: torch.Tensor):
        B, S, H = hidden_states.shape
        h = hidden_states.reshape(B * S, H)
        idx, w, _ = glm_route(h, self.weight, self.top_k, bias=self.selection_bias,
                              scaling=self.routed_scaling_factor, n_group=self.n_group,
                              topk_group=self.topk_group, norm_topk_prob=self.norm_topk_prob)
        return idx, w.to(hidden_states.dtype)

"""MoE layers over the grouped gfx950 INT4 kernels.

``moe_experts_forward`` replaces the per-expert Python loop of
MixtralMoELayer.forward (model/mixtral.py:290-370) and GLM4MoELayer.forward
(model/glm4.py:385-473):

  reference (per layer)                     here (per layer, no host sync)
  unique().tolist()          (D2H)          hn_moe_permute: counts, offsets, stable
  for e: where(idx == e)     (D2H x2)         permutation, active list (one WG)
         x[tok]; 4 launches                 hn_moe_gather: x_perm
         index_add_(fp16)                   hn_grouped_expert_mlp_int4: 2 launches over
                                              every active expert
                                            hn_moe_unpermute: fp16 index_add_ order

Expert weights come from a device table of slab pointers, one row per expert
(``ExpertTable``), built once when every expert is resident (fixed slots, or
a cache manager layer made resident in one HBM arena).  If a cache manager
holds only some experts, the active experts are fetched to the host (one
D2H), made resident through the manager (its get_int4_slot records
hits/misses and loads misses, none of them evicting another), and the table
is refreshed for that call.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import _lib
from .router import GLM4SigmoidRouter, TopKRouter, group_limit, router_logits


class ExpertTable:
    """Device table [E, 6] u64: gate_q, gate_s, up_q, up_s, down_q, down_s per expert."""

    def __init__(self, num_experts: int, device):
        self.num_experts = num_experts
        self.device = torch.device(device)
        self.host = torch.zeros((num_experts, 6), dtype=torch.int64)
        self.dev = torch.zeros((num_experts, 6), dtype=torch.int64, device=self.device)
        self.slots = [None] * num_experts
        self.dims = None

    def set(self, e: int, slot) -> None:
        dims = (slot.hidden_dim, slot.intermediate_dim, slot.group_size)
        if self.dims is None:
            self.dims = dims
        elif self.dims != dims:
            raise ValueError(f"expert {e} dims {dims} != table dims {self.dims}")
        ptrs = slot.data_ptrs()
        if any(p % 16 for p in ptrs):
            raise ValueError(f"expert {e}: weight and scale tensors must start 16-byte aligned")
        self.slots[e] = slot
        self.host[e] = torch.tensor(ptrs, dtype=torch.int64)

    def upload(self) -> None:
        self.dev.copy_(self.host)

    @classmethod
    def from_slots(cls, slots: Sequence, device=None) -> "ExpertTable":
        t = cls(len(slots), device or slots[0].device)
        for e, s in enumerate(slots):
            t.set(e, s)
        t.upload()
        return t


class Routed:
    """Routing of one MoE layer call: idx [T,k] i32, w [T,k] fp16, logits [T,E] f32
    (or None), the permutation metadata and the permuted rows x_perm [T*k, H]."""

    def __init__(self, T, k, E, H, device):
        n = max(T * k, 1)
        self.T, self.k, self.E = T, k, E
        self.meta = torch.empty(3 * E + 2 + 2 * n, dtype=torch.int32, device=device)
        self.offsets = self.meta[: E + 1]
        self.active = self.meta[E + 1: 2 * E + 1]
        self.n_active = self.meta[2 * E + 1: 2 * E + 2]
        self.perm = self.meta[2 * E + 2: 2 * E + 2 + n]
        self.inv = self.meta[2 * E + 2 + n: 2 * E + 2 + 2 * n]
        self.idx = torch.empty((T, k), dtype=torch.int32, device=device)
        self.w = torch.empty((T, k), dtype=torch.float16, device=device)
        self.logits = None
        self.x_perm = torch.empty((n, H), dtype=torch.float16, device=device)


def route_fits(T: int, E: int, k: int) -> bool:
    """Whether hn_moe_route (one launch) covers this batch."""
    return 0 < T * E <= _lib.ROUTE_MAX_LOGITS and T * k <= _lib.ROUTE_MAX_ASSIGN and E <= 256


def moe_route(hidden: torch.Tensor, k: int, mode: int, gate_w: Optional[torch.Tensor] = None,
              logits: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
              eps: float = 1e-9, scaling: float = 1.0, want_logits: bool = True,
              usage: Optional[torch.Tensor] = None) -> Routed:
    """Logits (from gate_w, unless ``logits`` is given), top-k, permutation and
    gather in one launch (hn_moe_route).  mode 0: Mixtral softmax top-k over
    fp16-rounded logits of an fp16 gate; mode 1: GLM sigmoid top-k (fp32 gate).
    usage: optional int64 [E] counters; the launch adds each expert's routed
    rows (TopKRouter's usage counts)."""
    T, H = hidden.shape
    _lib.require_gpu(hidden)
    dev = hidden.device
    x = _lib.aligned_rows(hidden.to(torch.float16))
    E = (logits.shape[1] if logits is not None else gate_w.shape[0])
    r = Routed(T, k, E, H, dev)
    wptr, ldw, wdt = None, 0, 0
    lg_in = None
    if logits is not None:
        lg_in = logits.to(torch.float32).contiguous()
        r.logits = lg_in
    else:
        wdt = 0 if mode == 0 else 1
        ww = gate_w.to(torch.float16 if wdt == 0 else torch.float32)
        ww = _lib.aligned_rows(ww)
        wptr, ldw = ww, ww.stride(0)
        if want_logits:
            r.logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    b = None if bias is None else bias.to(device=dev, dtype=torch.float32).contiguous()
    out_logits = r.logits if lg_in is None else None
    _lib.call("hn_moe_route", _lib.ptr(x), x.stride(0), _lib.ptr(wptr), ldw, wdt,
              _lib.ptr(lg_in), _lib.ptr(b), T, E, H, k, mode, eps, scaling,
              _lib.ptr(out_logits), _lib.ptr(r.idx), _lib.ptr(r.w), _lib.ptr(r.offsets),
              _lib.ptr(r.perm), _lib.ptr(r.inv), _lib.ptr(r.active), _lib.ptr(r.n_active),
              _lib.ptr(_usage_ptr(usage, E, dev)), _lib.ptr(r.x_perm), H, _lib.stream(dev))
    return r


def route_experts_fits(T: int, E: int, k: int, mode: int, table: "ExpertTable") -> bool:
    """Whether hn_moe_route_experts_decode (routing from given logits fused
    into the gate/up kernel) covers this layer call."""
    H, I, g = table.dims
    if table.num_experts != E:
        return False
    return _lib.lib().hn_moe_route_experts_decode_check(T, E, k, mode, H, I, g) == 0


def moe_route_experts_decode(hidden: torch.Tensor, logits: torch.Tensor, k: int, mode: int,
                             table: "ExpertTable", bias: Optional[torch.Tensor] = None,
                             eps: float = 1e-9, scaling: float = 1.0,
                             shared: Optional[torch.Tensor] = None, shared_ready=None,
                             usage: Optional[torch.Tensor] = None):
    """A decode MoE layer from given logits [T, E] in three launches
    (hn_moe_route_experts_decode): top-k and permutation inside the gate/up
    kernel, down projection, ordered unpermute (+ the fp16 shared addend once
    ``shared_ready``, a torch.cuda.Event recorded after it on another stream,
    has fired).  Returns (out [T, H] fp16, Routed without x_perm)."""
    T, H = hidden.shape
    _lib.require_gpu(hidden, logits)
    dev = hidden.device
    E = logits.shape[1]
    Ht, I, g = table.dims
    assert Ht == H, f"hidden {H} != expert hidden {Ht}"
    x = _lib.aligned_rows(hidden.to(torch.float16))
    r = Routed(T, k, E, 0, dev)
    r.logits = logits.to(torch.float32).contiguous()
    b = None if bias is None else bias.to(device=dev, dtype=torch.float32).contiguous()
    n = T * k
    h_ws = torch.empty((n, I), dtype=torch.float16, device=dev)
    y_ws = torch.empty((n, H), dtype=torch.float16, device=dev)
    sh = None if shared is None else _lib.aligned_rows(shared.reshape(T, H).to(torch.float16))
    out = torch.empty((T, H), dtype=torch.float16, device=dev)
    work = _lib.skinny_workspace(3, n, H, I, E, dev)
    ev = None if shared_ready is None else ctypes.c_void_p(shared_ready.cuda_event)
    _lib.call("hn_moe_route_experts_decode", _lib.ptr(r.logits), _lib.ptr(b), T, E, k, mode, eps,
              scaling, _lib.ptr(x), x.stride(0), _lib.ptr(table.dev), H, I, g, _lib.ptr(r.idx),
              _lib.ptr(r.w), _lib.ptr(r.offsets), _lib.ptr(r.perm), _lib.ptr(r.inv),
              _lib.ptr(r.active), _lib.ptr(r.n_active), _lib.ptr(_usage_ptr(usage, E, dev)),
              _lib.ptr(h_ws), _lib.ptr(y_ws), ev, _lib.ptr(sh),
              H if sh is None else sh.stride(0), _lib.ptr(out), H, _lib.ptr(work), work.numel(),
              _lib.stream(dev))
    return out, r


def moe_dispatch_joined(r: Routed, table: ExpertTable, shared: torch.Tensor,
                        shared_ready) -> torch.Tensor:
    """moe_dispatch with the fp16 shared addend produced on another stream:
    the expert kernels are queued first and the stream waits for
    ``shared_ready`` (a torch.cuda.Event recorded after the addend) only
    before the unpermute.  Down projections that run as K slices keep the
    one-call path (joined before it)."""
    T, k, E = r.T, r.k, r.E
    H = r.x_perm.shape[1]
    Ht, I, g = table.dims
    dev = r.x_perm.device
    n = T * k
    if T > _lib.DECODE_MAX_ROWS or I % 512 == 0:
        torch.cuda.current_stream(dev).wait_event(shared_ready)
        return moe_dispatch(r, table, shared=shared)
    st = _lib.stream(dev)
    h_ws = torch.empty((max(n, 1), I), dtype=torch.float16, device=dev)
    y_perm = torch.empty((max(n, 1), H), dtype=torch.float16, device=dev)
    out = torch.empty((T, H), dtype=torch.float16, device=dev)
    work = _lib.skinny_workspace(3, n, H, I, E, dev)
    _lib.call("hn_grouped_expert_mlp_int4", _lib.ptr(r.x_perm), _lib.ptr(table.dev),
              _lib.ptr(r.active), _lib.ptr(r.n_active), _lib.ptr(r.offsets), E, T, n, H, I, g,
              _lib.ptr(h_ws), _lib.ptr(y_perm), _lib.ptr(work), work.numel(), st)
    torch.cuda.current_stream(dev).wait_event(shared_ready)
    sh = _lib.aligned_rows(shared.reshape(T, H).to(torch.float16))  # after the wait
    _lib.call("hn_moe_unpermute", _lib.ptr(y_perm), H, _lib.ptr(r.inv), _lib.ptr(r.idx),
              _lib.ptr(r.w), T, k, _lib.ptr(sh), sh.stride(0), _lib.ptr(out), H, H, st)
    return out


def _usage_ptr(usage: Optional[torch.Tensor], E: int, dev) -> Optional[torch.Tensor]:
    if usage is None:
        return None
    assert usage.dtype == torch.int64 and usage.is_contiguous() and usage.numel() == E \
        and usage.device == torch.device(dev), "usage: contiguous int64 [E] on the layer's device"
    return usage


def decode_layer_fits(T: int, E: int, k: int, table: "ExpertTable", gate_w: torch.Tensor,
                      has_logits: bool = False) -> bool:
    """Whether hn_moe_decode_layer (routing fused into the gate/up kernel)
    covers this Mixtral layer call; has_logits: the router logits are given
    (then up to 64 routed rows, else up to 16 tokens)."""
    H, I, g = table.dims
    if table.num_experts != E or tuple(gate_w.shape) != (E, H):
        return False
    return _lib.lib().hn_moe_decode_layer_check(T, E, k, H, I, g, int(has_logits)) == 0


def experts_split_fits(T: int, k: int, table: "ExpertTable") -> bool:
    """Whether moe_dispatch at decode takes the streaming path with the K-split
    down projection (then it can fold the next RMSNorm into its unpermute)."""
    H, I, g = table.dims
    return T <= _lib.DECODE_MAX_ROWS and _lib.lib().hn_moe_experts_decode_split_check(
        table.num_experts, T, T * k, H, I, g) == 0


def _unpermute_add_rmsnorm(work: torch.Tensor, r: "Routed", H: int, I: int, fold):
    """(x + moe, RMSNorm(x + moe) * weight) from the down projection's fp32
    K-slice partials left in ``work`` (hn_unpermute_add_rmsnorm)."""
    T, k, E = r.T, r.k, r.E
    dev = work.device
    xr, nw, eps = fold
    xr = _lib.aligned_rows(xr.reshape(T, H))
    x_out = torch.empty((T, H), dtype=torch.float16, device=dev)
    h_out = torch.empty((T, H), dtype=torch.float16, device=dev)
    part = work.data_ptr() + _lib.lib().hn_moe_decode_layer_partials(T, E, k, H, I)
    _lib.call("hn_unpermute_add_rmsnorm", part, T * k * H, H, _lib.ptr(r.inv), _lib.ptr(r.idx),
              _lib.ptr(r.w), T, k, _lib.ptr(xr), xr.stride(0), _lib.ptr(x_out), H,
              _lib.ptr(nw), _lib.ptr(h_out), H, H, float(eps), _lib.stream(dev))
    return x_out, h_out


def moe_decode_layer(hidden: torch.Tensor, gate_w: torch.Tensor, k: int, table: "ExpertTable",
                     want_logits: bool = False, logits: Optional[torch.Tensor] = None,
                     usage: Optional[torch.Tensor] = None, fold=None):
    """One Mixtral MoE layer at decode in three launches (hn_moe_decode_layer):
    softmax top-k and the stable permutation computed in the gate/up kernel
    (with the fp16 gate logits, unless ``logits`` [T, E] are given), the down
    projection, the ordered weighted unpermute.  Returns (out [T, H] fp16,
    Routed) with the same routing outputs as moe_route (x_perm is not
    written).  fold = (x [T, H] fp16, norm weight [H] fp16, eps): the
    unpermute also adds the residual stream x and applies the next RMSNorm
    (hn_unpermute_add_rmsnorm); out is then (x + moe, RMSNorm(x + moe))."""
    T, H = hidden.shape
    _lib.require_gpu(hidden)
    dev = hidden.device
    E = gate_w.shape[0]
    Ht, I, g = table.dims
    assert Ht == H, f"hidden {H} != expert hidden {Ht}"
    x = _lib.aligned_rows(hidden.to(torch.float16))
    ww = _lib.aligned_rows(gate_w.to(torch.float16))
    r = Routed(T, k, E, 0, dev)
    lg_in = None
    if logits is not None:
        assert tuple(logits.shape) == (T, E), f"logits {tuple(logits.shape)} vs ({T}, {E})"
        lg_in = logits.to(torch.float32).contiguous()
        r.logits = lg_in
    elif want_logits:
        r.logits = torch.empty((T, E), dtype=torch.float32, device=dev)
    n = T * k
    h_ws = torch.empty((n, I), dtype=torch.float16, device=dev)
    out = torch.empty((T, H), dtype=torch.float16, device=dev) if fold is None else None
    work = _lib.skinny_workspace(3, n, H, I, E, dev)
    _lib.call("hn_moe_decode_layer", _lib.ptr(x), x.stride(0), _lib.ptr(ww), ww.stride(0),
              _lib.ptr(lg_in), T, E, k, _lib.ptr(table.dev), H, I, g, 1e-9, 1.0,
              _lib.ptr(r.logits if lg_in is None else None), _lib.ptr(r.idx),
              _lib.ptr(r.w), _lib.ptr(r.offsets), _lib.ptr(r.perm), _lib.ptr(r.inv),
              _lib.ptr(r.active), _lib.ptr(r.n_active), _lib.ptr(_usage_ptr(usage, E, dev)),
              _lib.ptr(h_ws), _lib.ptr(out), H,
              _lib.ptr(work), work.numel(), _lib.stream(dev))
    if fold is None:
        return out, r
    return _unpermute_add_rmsnorm(work, r, H, I, fold), r


def moe_dispatch(r: Routed, table: ExpertTable,
                 shared: Optional[torch.Tensor] = None, fold=None):
    """Grouped SwiGLU over the routed rows and the weighted, ordered sum back
    per token (the compute and unpermute halves of moe_experts_forward).
    fold = (x [T, H] fp16, norm weight [H] fp16, eps), only where
    experts_split_fits and without a shared expert: the unpermute also adds
    the residual stream x and applies the next RMSNorm; returns (x + moe,
    RMSNorm(x + moe))."""
    T, k, E = r.T, r.k, r.E
    H = r.x_perm.shape[1]
    Ht, I, g = table.dims
    assert Ht == H, f"hidden {H} != expert hidden {Ht}"
    assert table.num_experts == E, f"routing over {E} experts, table has {table.num_experts}"
    dev = r.x_perm.device
    st = _lib.stream(dev)
    n = T * k
    h_ws = torch.empty((max(n, 1), I), dtype=torch.float16, device=dev)
    y_perm = torch.empty((max(n, 1), H), dtype=torch.float16, device=dev)
    sh = None
    if shared is not None:
        sh = _lib.aligned_rows(shared.reshape(T, H).to(torch.float16))
    assert fold is None or (shared is None and T <= _lib.DECODE_MAX_ROWS), \
        "moe_dispatch: fold needs the decode path and no shared expert"
    out = torch.empty((T, H), dtype=torch.float16, device=dev) if fold is None else None
    if T <= _lib.DECODE_MAX_ROWS:
        # decode: both expert phases and the unpermute (split down projection)
        work = _lib.skinny_workspace(3, n, H, I, E, dev)
        _lib.call("hn_moe_experts_decode", _lib.ptr(r.x_perm), _lib.ptr(table.dev),
                  _lib.ptr(r.active), _lib.ptr(r.n_active), _lib.ptr(r.offsets), E, T, n, H, I,
                  g, _lib.ptr(h_ws), _lib.ptr(y_perm), _lib.ptr(r.inv), _lib.ptr(r.idx),
                  _lib.ptr(r.w), T, k, _lib.ptr(sh), H if sh is None else sh.stride(0),
                  _lib.ptr(out), H, _lib.ptr(work), work.numel(), st)
        return out if fold is None else _unpermute_add_rmsnorm(work, r, H, I, fold)
    work = _lib.gemm_workspace(dev)  # stream-K split of the prefill GEMM
    _lib.call("hn_grouped_expert_mlp_int4", _lib.ptr(r.x_perm), _lib.ptr(table.dev),
              _lib.ptr(r.active), _lib.ptr(r.n_active), _lib.ptr(r.offsets), E, T, n, H, I, g,
              _lib.ptr(h_ws), _lib.ptr(y_perm), _lib.ptr(work),
              0 if work is None else work.numel(), st)
    _lib.call("hn_moe_unpermute", _lib.ptr(y_perm), H, _lib.ptr(r.inv), _lib.ptr(r.idx),
              _lib.ptr(r.w), T, k, _lib.ptr(sh), H if sh is None else sh.stride(0), _lib.ptr(out),
              H, H, st)
    return out


def moe_experts_forward(hidden: torch.Tensor, idx: torch.Tensor, w: torch.Tensor,
                        table: ExpertTable, shared: Optional[torch.Tensor] = None) -> torch.Tensor:
    """out[T, H] = (shared +) sum_k w[t, k] * expert_{idx[t, k]}(hidden[t]).

    hidden [T, H] fp16; idx [T, k] int32; w [T, k] fp16; all on the GPU.
    Accumulation follows the reference: per expert fp16(y * w), added in
    ascending expert order into an fp16 buffer."""
    _lib.require_gpu(hidden, idx, w)
    T, H = hidden.shape
    k = idx.shape[1]
    E = table.num_experts
    Ht, I, g = table.dims
    assert Ht == H, f"hidden {H} != expert hidden {Ht}"
    dev = hidden.device
    st = _lib.stream(dev)
    x = _lib.aligned_rows(hidden.to(torch.float16))
    idx32 = idx.to(torch.int32).contiguous()
    wt = w.to(torch.float16).contiguous()
    n = T * k
    meta = torch.empty(3 * E + 2 + 2 * max(n, 1), dtype=torch.int32, device=dev)
    offsets = meta[: E + 1]
    active = meta[E + 1: 2 * E + 1]
    n_active = meta[2 * E + 1: 2 * E + 2]
    perm = meta[2 * E + 2: 2 * E + 2 + max(n, 1)]
    inv = meta[2 * E + 2 + max(n, 1): 2 * E + 2 + 2 * max(n, 1)]
    _lib.call("hn_moe_permute", _lib.ptr(idx32), T, k, E, _lib.ptr(offsets), _lib.ptr(perm),
              _lib.ptr(inv), _lib.ptr(active), _lib.ptr(n_active), st)
    x_perm = torch.empty((max(n, 1), H), dtype=torch.float16, device=dev)
    _lib.call("hn_moe_gather", _lib.ptr(x), x.stride(0), _lib.ptr(perm), k, _lib.ptr(offsets), E,
              _lib.ptr(x_perm), H, n, H, st)
    h_ws = torch.empty((max(n, 1), I), dtype=torch.float16, device=dev)
    y_perm = torch.empty((max(n, 1), H), dtype=torch.float16, device=dev)
    # above DECODE_MAX_ROWS tokens the grouped prefill GEMM runs, its workspace
    # holding the stream-K counters and partial sums
    work = (_lib.skinny_workspace(3, n, H, I, E, dev) if T <= _lib.DECODE_MAX_ROWS
            else _lib.gemm_workspace(dev))
    _lib.call("hn_grouped_expert_mlp_int4", _lib.ptr(x_perm), _lib.ptr(table.dev),
              _lib.ptr(active), _lib.ptr(n_active), _lib.ptr(offsets), E, T, n, H, I, g,
              _lib.ptr(h_ws), _lib.ptr(y_perm), _lib.ptr(work),
              0 if work is None else work.numel(), st)
    out = torch.empty((T, H), dtype=torch.float16, device=dev)
    sh = None
    if shared is not None:
        sh = _lib.aligned_rows(shared.reshape(T, H).to(torch.float16))
    _lib.call("hn_moe_unpermute", _lib.ptr(y_perm), H, _lib.ptr(inv), _lib.ptr(idx32),
              _lib.ptr(wt), T, k, _lib.ptr(sh), H if sh is None else sh.stride(0), _lib.ptr(out), H,
              H, st)
    return out


class _ResidentExperts:
    """Expert source for a layer: fixed slots, or a cache manager (offload case)."""

    def __init__(self, num_experts: int, layer_idx: int, slots=None, cache_manager=None):
        self.num_experts = num_experts
        self.layer_idx = layer_idx
        self.cache_manager = cache_manager
        self.table: Optional[ExpertTable] = None
        self._resident_table: Optional[ExpertTable] = None
        if slots is not None:
            self.table = ExpertTable.from_slots(slots)

    def static_table(self, device) -> Optional[ExpertTable]:
        """The table when it does not depend on the routing (fixed slots, or a
        cache manager holding every expert of the layer), else None."""
        cm = self.cache_manager
        if cm is None:
            return self.table
        if cm.is_resident(self.layer_idx):
            if self._resident_table is None:
                self._resident_table = ExpertTable.from_slots(cm.resident_slots(self.layer_idx),
                                                              device)
            return self._resident_table
        return None

    def table_for(self, idx: torch.Tensor) -> ExpertTable:
        cm = self.cache_manager
        if cm is None:
            return self.table
        if cm.is_resident(self.layer_idx):
            # every expert sits in the layer's HBM arena: static table, no host sync
            if self._resident_table is None:
                self._resident_table = ExpertTable.from_slots(cm.resident_slots(self.layer_idx),
                                                              idx.device)
            return self._resident_table
        if self.table is None:
            self.table = ExpertTable(self.num_experts, idx.device)
        needed = torch.unique(idx).tolist()  # one D2H when experts may be missing
        hits = [e for e in needed if cm.is_cached(self.layer_idx, e)]
        misses = [e for e in needed if e not in hits]
        # the experts of this call are used by one grouped launch: none may evict another
        with cm.hold(self.layer_idx, needed):
            for e in misses:  # start the loads of misses before touching hits
                cm.prefetch_int4_slot(self.layer_idx, e)
            for e in hits:
                self.table.set(e, cm.get_int4_slot(self.layer_idx, e))
            for e in misses:
                self.table.set(e, cm.get_int4_slot(self.layer_idx, e, prefetched_miss=True))
        self.table.upload()
        return self.table


class MixtralMoELayer(nn.Module):
    """Mixtral sparse-MoE block (model/mixtral.py:232-370) on the grouped kernels."""

    def __init__(self, hidden_dim: int = 4096, num_experts: int = 8, experts_per_token: int = 2,
                 layer_idx: int = 0, slots=None, cache_manager=None,
                 enable_affinity_bonus: Optional[bool] = None):
        super().__init__()
        self.layer_idx = layer_idx
        self.num_experts = num_experts
        # the cache-affinity bonus follows the cache manager's config, as the
        # reference's router reads ExpertCacheConfig (on by default,
        # config.py:273-275); without a cache manager there is nothing to favour
        cc = getattr(cache_manager, "cache_config", None)
        if enable_affinity_bonus is None:
            enable_affinity_bonus = bool(cc.enable_affinity_bonus) if cc is not None else False
        kw = {}
        if cc is not None:
            kw = dict(affinity_bonus=cc.affinity_bonus,
                      entropy_threshold=cc.affinity_entropy_threshold)
        self.router = TopKRouter(hidden_dim, num_experts, experts_per_token,
                                 enable_affinity_bonus=enable_affinity_bonus, **kw)
        self.experts = _ResidentExperts(num_experts, layer_idx, slots, cache_manager)
        if cache_manager is not None:
            self.router.set_cache_checker(lambda e: cache_manager.is_cached(layer_idx, e))
        # (idx [T, k] int32, w [T, k] fp16) of the last forward, on the device
        self.last_routing = None

    def takes_logits(self, T: int, top_k: int) -> bool:
        """Whether a forward of T tokens can take its router logits from the
        caller (e.g. hn_add_rmsnorm_router), saving the gate product: the
        one-launch routing and the decode layer with routing in its gate/up
        kernel both take them; past those sizes the router runs alone."""
        E, gw = self.num_experts, self.router.gate.weight
        return route_fits(T, E, top_k) and E <= 16 and gw.is_cuda

    def forward(self, hidden_states: torch.Tensor, top_k: int = 2,
                logits: Optional[torch.Tensor] = None) -> torch.Tensor:
        """logits: optional router logits [T, E] of hidden_states (fp16 values
        in fp32, as TopKRouter's gate Linear gives), used in place of the gate
        product where the routing takes them (takes_logits)."""
        B, S, H = hidden_states.shape
        T = B * S
        flat = hidden_states.reshape(T, H)
        rt = self.router
        if route_fits(T, self.num_experts, top_k):
            if rt.enable_affinity_bonus and rt._is_cached_fn is not None:
                if logits is None:
                    logits = router_logits(flat, rt.gate.weight.to(torch.float16))
                logits = rt._affinity(logits)
            table = self.experts.static_table(flat.device)
            # the routing launch adds to the usage counts (no host sync:
            # graph-capturable)
            usage = None if rt.training else rt.usage_counts
            if table is not None and decode_layer_fits(T, self.num_experts, top_k, table,
                                                       rt.gate.weight, logits is not None):
                # decode, resident experts: routing inside the gate/up kernel
                out, r = moe_decode_layer(flat, rt.gate.weight, top_k, table, logits=logits,
                                          usage=usage)
            else:
                # decode: routing, permutation and gather in one launch
                r = moe_route(flat, top_k, 0, gate_w=rt.gate.weight, logits=logits, usage=usage)
                out = moe_dispatch(r, self.experts.table_for(r.idx))
            self.last_routing = (r.idx, r.w)
            return out.view(B, S, H)
        ro = rt(hidden_states, top_k_override=top_k)
        idx = ro.expert_indices.reshape(T, top_k)
        w = ro.expert_weights.reshape(T, top_k)
        table = self.experts.table_for(idx)
        out = moe_experts_forward(flat, idx, w, table)
        self.last_routing = (idx, w)
        return out.view(B, S, H)

    def forward_folded(self, hidden_states: torch.Tensor, top_k: int,
                       logits: Optional[torch.Tensor], x: torch.Tensor, norm_weight: torch.Tensor,
                       eps: float):
        """The decode layer with the next RMSNorm folded into its last launch:
        returns (x + moe(hidden_states), RMSNorm(x + moe) * norm_weight) [B,
        S, H], bit-identical to forward() followed by the residual add and
        RMSNorm, or None where the folded launch does not apply (the caller
        then runs those two steps)."""
        B, S, H = hidden_states.shape
        T = B * S
        rt = self.router
        if not (hidden_states.is_cuda and route_fits(T, self.num_experts, top_k)):
            return None
        if rt.enable_affinity_bonus and rt._is_cached_fn is not None:
            return None
        table = self.experts.static_table(hidden_states.device)
        if table is None or norm_weight.dtype != torch.float16 or x.dtype != torch.float16:
            return None
        usage = None if rt.training else rt.usage_counts
        flat = hidden_states.reshape(T, H)
        fold = (x, norm_weight, eps)
        if decode_layer_fits(T, self.num_experts, top_k, table, rt.gate.weight,
                             logits is not None):
            (x_out, h_out), r = moe_decode_layer(flat, rt.gate.weight, top_k, table,
                                                 logits=logits, usage=usage, fold=fold)
        elif table.num_experts == self.num_experts and experts_split_fits(T, top_k, table):
            # e.g. 64 tokens at top-2: the routing launch, then the experts
            # with the unpermute folded into the next RMSNorm
            r = moe_route(flat, top_k, 0, gate_w=rt.gate.weight, logits=logits, usage=usage)
            x_out, h_out = moe_dispatch(r, table, fold=fold)
        else:
            return None
        self.last_routing = (r.idx, r.w)
        return x_out.view(B, S, H), h_out.view(B, S, H)


_SIDE_STREAMS: dict = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """One extra stream per device (default priority) for work that overlaps
    the routing kernels."""
    key = torch.device(device).index if torch.device(device).index is not None else \
        torch.cuda.current_device()
    if key not in _SIDE_STREAMS:
        _SIDE_STREAMS[key] = torch.cuda.Stream(device=key)
    return _SIDE_STREAMS[key]


class GLM4DenseMLP(nn.Module):
    """fp16 dense SwiGLU (model/glm4.py:220-235); shared expert of GLM4MoELayer.

    At inference the gate and up projections run as one GEMM over their
    stacked weights: the two parameters are re-pointed into one [2I, H]
    buffer on first use (no second copy), so every later call reads it with
    a single launch; the SiLU and the product (two fp16 roundings, as
    F.silu(g) * u) are one launch too.  Same fp16 Linear / SiLU / product
    sequence as the reference; the stacked GEMM may pick another kernel than
    two separate ones (fp32 summation order inside a dot product)."""

    def __init__(self, hidden_dim: int, intermediate_dim: int):
        super().__init__()
        self.gate_proj = nn.Linear(hidden_dim, intermediate_dim, bias=False)
        self.up_proj = nn.Linear(hidden_dim, intermediate_dim, bias=False)
        self.down_proj = nn.Linear(intermediate_dim, hidden_dim, bias=False)
        self._stacked: Optional[torch.Tensor] = None

    def _gate_up_weight(self) -> Optional[torch.Tensor]:
        g, u = self.gate_proj, self.up_proj
        if type(g) is not nn.Linear or type(u) is not nn.Linear or g.bias is not None \
                or u.bias is not None:
            return None  # e.g. converted to Int4Linear
        wg, wu = g.weight, u.weight
        if torch.is_grad_enabled() and (wg.requires_grad or wu.requires_grad):
            return None
        st = self._stacked
        n = wg.shape[0]
        if st is not None and wg.data_ptr() == st.data_ptr() and \
                wu.data_ptr() == st[n:].data_ptr() and wg.shape == st[:n].shape and \
                wu.shape == st[n:].shape:
            return st
        if wg.dtype != wu.dtype or wg.device != wu.device or wg.shape[1] != wu.shape[1]:
            return None
        st = torch.cat([wg.detach(), wu.detach()], 0).contiguous()
        g.weight.data = st[:n]
        u.weight.data = st[n:]
        self._stacked = st
        return st

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w = self._gate_up_weight()
        if w is None or w.dtype != torch.float16 or not w.is_cuda:
            return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))
        n = self.gate_proj.out_features
        gu = F.linear(x, w).reshape(-1, 2 * n)
        h = torch.empty((gu.shape[0], n), dtype=torch.float16, device=gu.device)
        # fp16(fp16(silu(g)) * u): F.silu then the product, in one launch
        _lib.call("hn_silu_then_mul", _lib.ptr(gu), 2 * n, _lib.ptr(gu[:, n:]), 2 * n,
                  _lib.ptr(h), n, gu.shape[0], n, _lib.stream(gu.device))
        return self.down_proj(h.view(*x.shape[:-1], n))


class GLM4MoELayer(nn.Module):
    """GLM-4.5-Air MoE block (model/glm4.py:312-473): fp16 shared expert plus
    routed INT4 experts, out = shared + routed (fp16 add fused into unpermute)."""

    def __init__(self, hidden_dim: int = 4096, moe_intermediate_dim: int = 1408,
                 num_experts: int = 128, experts_per_token: int = 8, layer_idx: int = 0,
                 slots=None, cache_manager=None, routed_scaling_factor: float = 1.0,
                 num_shared_experts: int = 1, n_group: int = 1, topk_group: int = 1,
                 norm_topk_prob: bool = True):
        super().__init__()
        self.layer_idx = layer_idx
        self.router = GLM4SigmoidRouter(hidden_dim, num_experts, experts_per_token,
                                        norm_topk_prob=norm_topk_prob,
                                        routed_scaling_factor=routed_scaling_factor,
                                        n_group=n_group, topk_group=topk_group)
        # one dense MLP as wide as all the shared experts together
        # (model/glm4.py:341-344)
        self.shared_expert = GLM4DenseMLP(hidden_dim, moe_intermediate_dim * num_shared_experts)
        self.experts = _ResidentExperts(num_experts, layer_idx, slots, cache_manager)
        self._last_idx: Optional[torch.Tensor] = None
        self.last_routing = None  # (idx [T, k] i32, w [T, k] fp16) of the last forward
        # decode routing inside the gate/up kernel (hn_moe_route_experts_decode)
        # instead of the separate routing launch
        self.fused_routing = False
        # the shared expert on a second stream, overlapping the routing and
        # expert kernels (joined before the unpermute); False runs it first on
        # the layer's stream (measured at 32 tokens: 222.4 us per layer with
        # the side stream, 226-228 us without)
        self.shared_side_stream = True

    def get_last_selected_experts(self) -> list:
        """Experts the last forward routed to, ascending (the reference records
        unique(expert_indices) for the next layer's prefetch, model/glm4.py:469,
        704-713).  The forward keeps the indices on the device; the list is made
        here, so only a caller that asks pays the device-to-host copy."""
        if self._last_idx is None:
            return []
        return torch.unique(self._last_idx).tolist()

    def prefetch_predicted(self, predicted_experts) -> None:
        """Start the loads of predicted experts that are not resident
        (model/glm4.py:351-363): with a cache manager that holds only part of
        the layer, each miss is scheduled on the store's copy stream."""
        cm = self.experts.cache_manager
        if cm is None or cm.is_resident(self.layer_idx):
            return
        for e in predicted_experts:
            if not cm.is_cached(self.layer_idx, int(e)):
                cm.prefetch_int4_slot(self.layer_idx, int(e))

    def forward(self, hidden_states: torch.Tensor, skip_routed: bool = False) -> torch.Tensor:
        B, S, H = hidden_states.shape
        if skip_routed:
            return self.shared_expert(hidden_states)
        T = B * S
        flat = hidden_states.reshape(T, H)
        rt = self.router
        mode = 1 if rt.norm_topk_prob else 2
        table = self.experts.static_table(flat.device)
        if self.fused_routing and table is not None and \
                route_experts_fits(T, rt.num_experts, rt.top_k, mode, table):
            # the shared expert (fp16 GEMMs) on a side stream, joined only
            # before the unpermute; the routing runs inside the gate/up kernel
            cur = torch.cuda.current_stream(flat.device)
            side = _side_stream(flat.device)
            side.wait_stream(cur)
            with torch.cuda.stream(side):
                shared = self.shared_expert(hidden_states)
                ready = torch.cuda.Event()
                ready.record(side)
            logits = router_logits(flat, rt.weight.float() if rt.weight.dtype != torch.float32
                                   else rt.weight)
            if rt.n_group > 1 and rt.topk_group > 0:
                logits = group_limit(logits, rt.n_group, rt.topk_group)
            out, r = moe_route_experts_decode(flat, logits, rt.top_k, mode, table,
                                              bias=rt.selection_bias,
                                              scaling=rt.routed_scaling_factor,
                                              shared=shared.reshape(T, H), shared_ready=ready)
            shared.record_stream(cur)
            self._last_idx = r.idx
            self.last_routing = (r.idx, r.w)
            return out.view(B, S, H)
        if route_fits(T, rt.num_experts, rt.top_k) and not self.shared_side_stream:
            # the shared expert first, on the same stream
            shared = self.shared_expert(hidden_states)
            logits = router_logits(flat, rt.weight.float() if rt.weight.dtype != torch.float32
                                   else rt.weight)
            if rt.n_group > 1 and rt.topk_group > 0:
                logits = group_limit(logits, rt.n_group, rt.topk_group)
            r = moe_route(flat, rt.top_k, mode, logits=logits,
                          bias=rt.selection_bias, scaling=rt.routed_scaling_factor)
            out = moe_dispatch(r, self.experts.table_for(r.idx), shared=shared.reshape(T, H))
            self._last_idx = r.idx
            self.last_routing = (r.idx, r.w)
            return out.view(B, S, H)
        if route_fits(T, rt.num_experts, rt.top_k):
            # the shared expert (fp16 GEMMs) runs on a side stream while the
            # router, the routing and the expert kernels run; joined before
            # the unpermute
            cur = torch.cuda.current_stream(flat.device)
            side = _side_stream(flat.device)
            side.wait_stream(cur)
            with torch.cuda.stream(side):
                shared = self.shared_expert(hidden_states)
                ready = torch.cuda.Event()
                ready.record(side)
            # fp32 logits by the multi-workgroup kernel, the rest in one launch
            logits = router_logits(flat, rt.weight.float() if rt.weight.dtype != torch.float32
                                   else rt.weight)
            if rt.n_group > 1 and rt.topk_group > 0:
                logits = group_limit(logits, rt.n_group, rt.topk_group)
            r = moe_route(flat, rt.top_k, mode, logits=logits,
                          bias=rt.selection_bias, scaling=rt.routed_scaling_factor)
            shared.record_stream(cur)
            out = moe_dispatch_joined(r, self.experts.table_for(r.idx), shared.reshape(T, H),
                                      ready)
            self._last_idx = r.idx
            self.last_routing = (r.idx, r.w)
            return out.view(B, S, H)
        shared = self.shared_expert(hidden_states)
        idx, w = rt(hidden_states)
        table = self.experts.table_for(idx)
        out = moe_experts_forward(flat, idx, w, table, shared=shared.reshape(T, H))
        self._last_idx = idx
        self.last_routing = (idx, w)
        return out.view(B, S, H)

"""Fused INT4 GEMM / SwiGLU expert MLP on gfx950 (HIP, via libhn_int4.so).

Drop-in for the reference module kernels/int4_gemm.py: the same three public
functions with the same signatures, argument meaning, output allocation and
AssertionError shape checks.  The Triton kernels are replaced by hand-written
HIP kernels behind the C ABI in include/hn_int4.h:

* ``int4_linear``            -> ``hn_int4_linear``        (kernels/int4_gemm.py:124-172)
* ``fused_silu_mul``         -> ``hn_silu_mul``           (kernels/int4_gemm.py:196-208)
* ``expert_mlp_int4_fused``  -> ``hn_expert_mlp_int4``    (kernels/int4_gemm.py:211-254):
  gate, up and SiLU*up in one launch, down in a second; the [T, I] fp16
  intermediate is the only activation buffer.

Numerics: fp16 in/out, fp32 accumulation, gate/up rounded to fp16 before the
SiLU product, as in the reference.  There is no CPU path.
"""
from __future__ import annotations

import torch

from .. import _lib


def _as_f16(x: torch.Tensor) -> torch.Tensor:
    return x if x.dtype == torch.float16 else x.to(torch.float16)


def int4_linear(
    x: torch.Tensor,           # [M, K] or [batch, seq, K] fp16
    w_packed: torch.Tensor,    # [N, K//2] uint8
    w_scales: torch.Tensor,    # [N, K//group_size] fp16
    group_size: int = 128,
) -> torch.Tensor:
    """out = x @ W.T with W stored as INT4 + per-group fp16 scales, dequantised in
    registers (no fp16 weight materialisation).  Output dtype is x.dtype."""
    orig_shape = x.shape
    if x.dim() == 3:
        batch, seq, K = x.shape
        x = x.reshape(batch * seq, K)

    M, K = x.shape
    N = w_packed.shape[0]

    assert w_packed.shape[1] == K // 2, f"w_packed shape {w_packed.shape} vs K={K}"
    assert w_scales.shape == (N, K // group_size), \
        f"w_scales shape {w_scales.shape} vs ({N}, {K // group_size})"

    _lib.require_gpu(x, w_packed, w_scales)
    out_dtype = x.dtype
    xh = _lib.aligned_rows(_as_f16(x))
    wq = _lib.aligned_rows(w_packed)
    ws = w_scales if w_scales.stride(-1) == 1 else w_scales.contiguous()
    out = torch.empty((M, N), dtype=torch.float16, device=x.device)
    work = (_lib.skinny_workspace(0, M, N, K, 0, x.device) if M <= _lib.DECODE_MAX_ROWS
            else _lib.gemm_workspace(x.device))
    _lib.call("hn_int4_linear", _lib.ptr(xh), xh.stride(0), _lib.ptr(wq), wq.stride(0),
              _lib.ptr(ws), ws.stride(0), _lib.ptr(out), out.stride(0), M, N, K, group_size,
              _lib.ptr(work), work.numel(), _lib.stream(x.device))
    if out_dtype != torch.float16:
        out = out.to(out_dtype)
    if len(orig_shape) == 3:
        out = out.view(batch, seq, N)
    return out


def fused_silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """fp16(silu(float(gate)) * float(up)), elementwise."""
    assert gate.shape == up.shape
    _lib.require_gpu(gate, up)
    g = gate.contiguous()
    u = up.contiguous()
    out = torch.empty_like(g)
    n = g.numel()
    if n == 0:
        return out
    cols = g.shape[-1] if g.dim() > 0 else 1
    rows = n // cols
    _lib.call("hn_silu_mul", _lib.ptr(g), cols, _lib.ptr(u), cols, _lib.ptr(out), cols, rows, cols,
              _lib.stream(g.device))
    return out


def expert_mlp_int4_fused(
    x: torch.Tensor,              # [num_tokens, hidden_dim] fp16
    gate_packed: torch.Tensor,    # [intermediate_dim, hidden_dim//2] uint8
    gate_scales: torch.Tensor,    # [intermediate_dim, hidden_dim//group_size] fp16
    up_packed: torch.Tensor,      # [intermediate_dim, hidden_dim//2] uint8
    up_scales: torch.Tensor,      # [intermediate_dim, hidden_dim//group_size] fp16
    down_packed: torch.Tensor,    # [hidden_dim, intermediate_dim//2] uint8
    down_scales: torch.Tensor,    # [hidden_dim, intermediate_dim//group_size] fp16
    group_size: int = 128,
) -> torch.Tensor:
    """out = down(silu(gate(x)) * up(x)) with INT4 weights, no fp16 weights."""
    orig_shape = x.shape
    if x.dim() == 3:
        x = x.reshape(-1, x.shape[-1])
    T, H = x.shape
    I = gate_packed.shape[0]
    assert gate_packed.shape[1] == H // 2, f"w_packed shape {gate_packed.shape} vs K={H}"
    assert gate_scales.shape == (I, H // group_size), \
        f"w_scales shape {gate_scales.shape} vs ({I}, {H // group_size})"
    assert up_packed.shape[1] == H // 2, f"w_packed shape {up_packed.shape} vs K={H}"
    assert up_scales.shape == (up_packed.shape[0], H // group_size), \
        f"w_scales shape {up_scales.shape} vs ({up_packed.shape[0]}, {H // group_size})"
    assert up_packed.shape[0] == I, "gate and up projections must have the same rows"
    assert down_packed.shape == (H, I // 2), f"w_packed shape {down_packed.shape} vs K={I}"
    assert down_scales.shape == (H, I // group_size), \
        f"w_scales shape {down_scales.shape} vs ({H}, {I // group_size})"

    _lib.require_gpu(x, gate_packed, gate_scales, up_packed, up_scales, down_packed, down_scales)
    out_dtype = x.dtype
    xh = _as_f16(x)
    if xh.stride(-1) != 1 or xh.stride(0) != H or xh.data_ptr() % 16:
        xh = xh.contiguous()
        if xh.data_ptr() % 16:
            xh = xh.clone()
    mats = [t.contiguous() for t in (gate_packed, gate_scales, up_packed, up_scales, down_packed,
                                     down_scales)]
    h_ws = torch.empty((T, I), dtype=torch.float16, device=x.device)
    out = torch.empty((T, H), dtype=torch.float16, device=x.device)
    if T > 0:
        work = (_lib.skinny_workspace(2, T, H, I, 0, x.device) if T <= _lib.DECODE_MAX_ROWS
                else _lib.gemm_workspace(x.device))
        _lib.call("hn_expert_mlp_int4", _lib.ptr(xh), *[_lib.ptr(m) for m in mats], _lib.ptr(out),
                  T, H, I, group_size, _lib.ptr(h_ws), _lib.ptr(work), work.numel(),
                  _lib.stream(x.device))
    if out_dtype != torch.float16:
        out = out.to(out_dtype)
    if len(orig_shape) == 3:
        out = out.view(*orig_shape[:-1], H)
    return out


def dequantize_int4(packed: torch.Tensor, scales: torch.Tensor, group_size: int = 128,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """fp16 [N, K] = fp16((nibble - 8) * scale), bit-exact with the reference's
    dequantisers (preprocess/pack_weights.py:230-268)."""
    _lib.require_gpu(packed, scales)
    N, Kh = packed.shape
    K = Kh * 2
    assert scales.shape == (N, K // group_size), \
        f"scales shape {scales.shape} vs ({N}, {K // group_size})"
    pq = _lib.aligned_rows(packed)
    sc = scales.contiguous()
    if out is None:
        out = torch.empty((N, K), dtype=torch.float16, device=packed.device)
    _lib.call("hn_int4_dequant", _lib.ptr(pq), pq.stride(0), _lib.ptr(sc), sc.stride(0),
              _lib.ptr(out), out.stride(0), N, K, group_size, _lib.stream(packed.device))
    return out


def quantize_int4(w: torch.Tensor, group_size: int = 128, mode: int = 0):
    """GPU quantiser.  mode 0 = ExpertWeightPacker.quantize_tensor
    (preprocess/pack_weights.py:133-181, fp16 input); mode 1 =
    Int4Linear.quantize_weight (kernels/int4_linear.py:68-107, fp16 or fp32).
    Returns (packed uint8 [N, K/2], scales fp16 [N, K/group]) on w's device."""
    _lib.require_gpu(w)
    N, K = w.shape
    assert K % group_size == 0, f"in_features {K} must be divisible by group_size {group_size}"
    assert K % 2 == 0
    if w.dtype not in (torch.float16, torch.float32):
        w = w.to(torch.float16 if mode == 0 else torch.float32)
    w = w.contiguous()
    packed = torch.empty((N, K // 2), dtype=torch.uint8, device=w.device)
    scales = torch.empty((N, K // group_size), dtype=torch.float16, device=w.device)
    dtype = 0 if w.dtype == torch.float16 else 1
    _lib.call("hn_int4_quantize", _lib.ptr(w), w.stride(0), dtype, mode, _lib.ptr(packed),
              packed.stride(0), _lib.ptr(scales), scales.stride(0), N, K, group_size,
              _lib.stream(w.device))
    return packed, scales

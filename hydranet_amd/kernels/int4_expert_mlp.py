"""INT4 expert MLP with the signatures of the reference's kernels/int4_expert_mlp.py.

Same functions, same shape checks (``int4_linear`` asserts the exact
``w_packed.shape == (N, K // 2)``, kernels/int4_expert_mlp.py:126-127), backed
by the gfx950 kernels of libhn_int4.so:

* ``int4_linear``               (kernels/int4_expert_mlp.py:99-156)  -> hn_int4_linear
* ``silu_mul``                  (:189-210)                           -> hn_silu_mul (2-D / 3-D)
* ``expert_mlp_int4``           (:213-252)                           -> hn_expert_mlp_int4
* ``expert_mlp_int4_from_slot`` (:255-272)                           reads gpu_slot.{gate,up,down}_{packed,scales}

x of any float dtype is read as fp16; the output has x's dtype, values rounded
through fp16 (the reference kernel casts x to fp16 on load and stores fp16).
"""
from __future__ import annotations

import torch

from . import int4_gemm as _g


def int4_linear(
    x: torch.Tensor,           # [M, K] fp16
    w_packed: torch.Tensor,    # [N, K//2] uint8
    w_scales: torch.Tensor,    # [N, K//group_size] fp16
    group_size: int = 128,
) -> torch.Tensor:
    orig_shape = x.shape
    if x.dim() == 3:
        batch, seq, K = x.shape
        x = x.reshape(batch * seq, K)
    M, K = x.shape
    N = w_packed.shape[0]
    assert w_packed.shape == (N, K // 2), \
        f"w_packed shape mismatch: {w_packed.shape} vs ({N}, {K // 2})"
    assert w_scales.shape == (N, K // group_size), \
        f"w_scales shape mismatch: {w_scales.shape} vs ({N}, {K // group_size})"
    out = _g.int4_linear(x, w_packed, w_scales, group_size)
    if len(orig_shape) == 3:
        out = out.view(batch, seq, N)
    return out


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Fused SiLU(gate) * up on 2-D or 3-D tensors."""
    assert gate.shape == up.shape
    return _g.fused_silu_mul(gate, up)


def expert_mlp_int4(
    x: torch.Tensor,
    gate_packed: torch.Tensor,
    gate_scales: torch.Tensor,
    up_packed: torch.Tensor,
    up_scales: torch.Tensor,
    down_packed: torch.Tensor,
    down_scales: torch.Tensor,
    group_size: int = 128,
) -> torch.Tensor:
    """out = down(silu(gate(x)) * up(x)), INT4 weights, no fp16 materialisation."""
    return _g.expert_mlp_int4_fused(x, gate_packed, gate_scales, up_packed, up_scales,
                                    down_packed, down_scales, group_size)


def expert_mlp_int4_from_slot(
    x: torch.Tensor,
    gpu_slot,  # GpuExpertSlot with INT4 buffers
    group_size: int = 128,
) -> torch.Tensor:
    return expert_mlp_int4(
        x,
        gpu_slot.gate_packed, gpu_slot.gate_scales,
        gpu_slot.up_packed, gpu_slot.up_scales,
        gpu_slot.down_packed, gpu_slot.down_scales,
        group_size,
    )

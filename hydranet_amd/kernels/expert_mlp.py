"""Expert MLP entry points with the names of the reference's kernels/expert_mlp.py.

The reference's ``ExpertMLPTriton.forward`` (kernels/expert_mlp.py:254-303)
dequantises all three projections to fp16 and runs torch matmuls; its Triton
kernels are never launched.  Here the class keeps its name and signature for
callers (package export ``expert_mlp_int4`` with ``hidden_dim`` and
``intermediate_dim`` arguments, kernels/__init__.py:15) but runs the fused
gfx950 INT4 kernel; ``_dequant`` is the bit-exact HIP dequantiser.
"""
from __future__ import annotations

import torch

from . import int4_gemm as _g


class ExpertMLPTriton:
    """SwiGLU expert MLP over INT4 weights (name kept from the reference)."""

    def __init__(self, hidden_dim: int, intermediate_dim: int, group_size: int = 128,
                 device: torch.device = torch.device("cuda")):
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.group_size = group_size
        self.device = device

    def forward(self, x, gate_packed, gate_scales, up_packed, up_scales, down_packed,
                down_scales) -> torch.Tensor:
        return _g.expert_mlp_int4_fused(x, gate_packed, gate_scales, up_packed, up_scales,
                                        down_packed, down_scales, self.group_size)

    __call__ = forward

    def _dequant(self, packed: torch.Tensor, scales: torch.Tensor, out_features: int,
                 in_features: int) -> torch.Tensor:
        assert packed.shape == (out_features, in_features // 2)
        return _g.dequantize_int4(packed, scales, self.group_size)


def expert_mlp_int4(x, gate_packed, gate_scales, up_packed, up_scales, down_packed, down_scales,
                    hidden_dim: int, intermediate_dim: int, group_size: int = 128) -> torch.Tensor:
    mlp = ExpertMLPTriton(hidden_dim, intermediate_dim, group_size, x.device)
    return mlp.forward(x, gate_packed, gate_scales, up_packed, up_scales, down_packed, down_scales)

"""INT4 Linear layer (reference: kernels/int4_linear.py:19-269), gfx950 forward.

Same module, buffer names (``weight_packed`` [out, in/2] uint8, ``weight_scale``
[out, in/group] fp16), fp16 bias, quantiser formula and group-size fallback as
the reference.  ``forward`` runs hn_int4_linear; ``quantize_weight`` runs the
mode-1 HIP quantiser, which restates Int4Linear.quantize_weight's arithmetic
(it differs from the expert packer's).  Tensors on a CPU device are moved to
the GPU for quantisation; the forward has no CPU path.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import int4_gemm as _g
from .int4_gemm import int4_linear


class Int4Linear(nn.Module):
    """Linear layer with INT4 weights, fp16 compute, optional fp16 bias."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 group_size: int = 128, device: Optional[torch.device] = None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.group_size = group_size
        assert in_features % group_size == 0, \
            f"in_features ({in_features}) must be divisible by group_size ({group_size})"
        assert in_features % 2 == 0, f"in_features ({in_features}) must be even for INT4 packing"
        num_groups = in_features // group_size
        self.register_buffer("weight_packed",
                             torch.zeros(out_features, in_features // 2, dtype=torch.uint8,
                                         device=device))
        self.register_buffer("weight_scale",
                             torch.ones(out_features, num_groups, dtype=torch.float16,
                                        device=device))
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.float16, device=device))
        else:
            self.register_parameter("bias", None)

    @staticmethod
    def quantize_weight(weight: torch.Tensor, group_size: int = 128):
        """(out, in) fp16/fp32 -> (packed (out, in//2) uint8, scale (out, in//g) fp16)."""
        out_features, in_features = weight.shape
        assert in_features % group_size == 0
        dev = weight.device
        w = weight.detach()
        if w.device.type != "cuda":
            w = w.to("cuda")
        packed, scale = _g.quantize_int4(w, group_size, mode=1)
        return packed.to(dev), scale.to(dev)

    @classmethod
    def from_float(cls, linear: nn.Linear, group_size: int = 128,
                   device: Optional[torch.device] = None) -> "Int4Linear":
        device = device or linear.weight.device
        in_features = linear.in_features
        if in_features % group_size != 0:
            group_size = 64
            if in_features % group_size != 0:
                group_size = 32
                if in_features % group_size != 0:
                    raise ValueError(
                        f"in_features ({in_features}) must be divisible by a power-of-2 group size")
        layer = cls(in_features=linear.in_features, out_features=linear.out_features,
                    bias=linear.bias is not None, group_size=group_size, device=device)
        weight_packed, scale = cls.quantize_weight(linear.weight.data, group_size)
        layer.weight_packed.copy_(weight_packed)
        layer.weight_scale.copy_(scale)
        if linear.bias is not None:
            layer.bias.data.copy_(linear.bias.data.to(torch.float16))
        return layer

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        out = int4_linear(x, self.weight_packed, self.weight_scale, self.group_size)
        if self.bias is not None:
            out = out + self.bias
        return out

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, dtype=int4, group_size={self.group_size}")


def convert_model_to_int4(model: nn.Module, skip_layers: Optional[list] = None,
                          group_size: int = 128, device: Optional[torch.device] = None) -> nn.Module:
    """Replace nn.Linear modules by Int4Linear in place (kernels/int4_linear.py:174-236)."""
    skip_layers = skip_layers or []

    def should_skip(name: str) -> bool:
        return any(skip in name for skip in skip_layers)

    converted = 0
    skipped = 0
    for name, module in list(model.named_modules()):
        if should_skip(name):
            skipped += 1
            continue
        if isinstance(module, nn.Linear):
            if module.in_features % 2 != 0:
                print(f"  Skipping {name}: in_features ({module.in_features}) not even")
                skipped += 1
                continue
            gs = group_size
            while gs > 1 and module.in_features % gs != 0:
                gs = gs // 2
            if gs < 32:
                print(f"  Skipping {name}: no compatible group size for "
                      f"in_features={module.in_features}")
                skipped += 1
                continue
            parts = name.rsplit(".", 1)
            if len(parts) == 1:
                parent, attr = model, parts[0]
            else:
                parent, attr = model.get_submodule(parts[0]), parts[1]
            setattr(parent, attr, Int4Linear.from_float(module, group_size=gs, device=device))
            converted += 1
    print(f"  Converted {converted} layers to INT4, skipped {skipped}")
    return model


def estimate_int4_memory(model: nn.Module, group_size: int = 128) -> dict:
    """fp16 vs INT4(+scales) parameter bytes (kernels/int4_linear.py:239-269)."""
    fp16_bytes = 0
    int4_bytes = 0
    for _, param in model.named_parameters():
        numel = param.numel()
        fp16_bytes += numel * 2
        if param.dim() == 2:
            out_features, in_features = param.shape
            int4_bytes += numel // 2
            num_groups = (in_features + group_size - 1) // group_size
            int4_bytes += out_features * num_groups * 2
        else:
            int4_bytes += numel * 2
    return {
        "fp16_mb": fp16_bytes / 1e6,
        "int4_mb": int4_bytes / 1e6,
        "savings_mb": (fp16_bytes - int4_bytes) / 1e6,
    }

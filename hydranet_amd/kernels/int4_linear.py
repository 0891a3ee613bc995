"""INT4 linear layers for a model's non-expert weights (attention projections,
a dense shared expert): the drop-in for HydraNet's ``Int4Linear`` and its
helpers (kernels/int4_linear.py:19-269).

Kept from the reference because callers and saved state depend on them:
the class and function names and arguments, the buffer names and layouts
(``weight_packed`` [out, in/2] uint8, low nibble = even input index;
``weight_scale`` [out, in/group] fp16; an fp16 ``bias`` parameter), the
quantiser's arithmetic (``quantize_weight``; it differs from the expert
packer's), the group-size choices of ``from_float`` (the requested group,
else 64, else 32) and of ``convert_model_to_int4`` (halve until it divides
``in_features``, give up below 32; here also passing over a group that is
not a multiple of 32, which the gfx950 kernels do not take), and the keys
and arithmetic of ``estimate_int4_memory``.

This build's part: quantisation runs on the GPU (the mode-1 HIP quantiser,
bit-exact with the reference's torch arithmetic), the forward is the gfx950
W4A16 kernel (``hn_int4_linear``: decode GEMV / prefill MFMA GEMM), and the
decoder harness stacks the q/k/v layers' packed weights into one launch
(``stacked_int4``).  There is no CPU forward.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence

import torch
import torch.nn as nn

from . import int4_gemm as _g

__all__ = ["Int4Linear", "convert_model_to_int4", "estimate_int4_memory", "stacked_int4"]

# group sizes from_float tries after the requested one
_FROM_FLOAT_FALLBACK = (64, 32)
# convert_model_to_int4 halves the group size down to this, then skips the layer
_MIN_GROUP = 32


def _group_for_from_float(in_features: int, group_size: int) -> int:
    for g in (group_size,) + _FROM_FLOAT_FALLBACK:
        if in_features % g == 0:
            return g
    raise ValueError(f"Int4Linear.from_float: no group size among "
                     f"{(group_size,) + _FROM_FLOAT_FALLBACK} divides in_features={in_features}")


def _group_for_convert(in_features: int, group_size: int) -> Optional[int]:
    # halving as the reference does; a group the W4A16 kernels do not take
    # (not a multiple of 32, e.g. 48 from 96) is passed over like one that
    # does not divide in_features
    g = group_size
    while g >= _MIN_GROUP:
        if in_features % g == 0 and g % 32 == 0:
            return g
        g //= 2
    return None


class Int4Linear(nn.Module):
    """y = x W^T (+ bias) with W held as INT4 nibbles and per-group fp16 scales."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 group_size: int = 128, device: Optional[torch.device] = None):
        super().__init__()
        assert in_features % 2 == 0, f"Int4Linear: in_features={in_features} is odd (two " \
                                     f"weights per byte)"
        assert in_features % group_size == 0, f"Int4Linear: group_size={group_size} does not " \
                                              f"divide in_features={in_features}"
        self.in_features, self.out_features, self.group_size = in_features, out_features, \
            group_size
        self.register_buffer("weight_packed", torch.zeros(
            (out_features, in_features // 2), dtype=torch.uint8, device=device))
        self.register_buffer("weight_scale", torch.ones(
            (out_features, in_features // group_size), dtype=torch.float16, device=device))
        self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.float16, device=device)) \
            if bias else None

    @staticmethod
    def quantize_weight(weight: torch.Tensor, group_size: int = 128):
        """[out, in] fp16 / fp32 -> (packed [out, in/2] uint8, scale [out, in/group] fp16),
        the reference's Int4Linear quantiser (kernels/int4_linear.py:68-107), run by the
        HIP quantiser on the GPU; results come back on weight's device."""
        assert weight.dim() == 2 and weight.shape[1] % group_size == 0, \
            f"quantize_weight: shape {tuple(weight.shape)} vs group_size={group_size}"
        home = weight.device
        w = weight.detach()
        packed, scale = _g.quantize_int4(w if w.is_cuda else w.cuda(), group_size, mode=1)
        return packed.to(home), scale.to(home)

    def load_quantized(self, packed: torch.Tensor, scale: torch.Tensor,
                       bias: Optional[torch.Tensor] = None) -> "Int4Linear":
        self.weight_packed.copy_(packed)
        self.weight_scale.copy_(scale)
        if self.bias is not None and bias is not None:
            with torch.no_grad():
                self.bias.copy_(bias.to(torch.float16))
        return self

    @classmethod
    def from_float(cls, linear: nn.Linear, group_size: int = 128,
                   device: Optional[torch.device] = None) -> "Int4Linear":
        """Quantise an nn.Linear; the group falls back to 64 then 32 when the
        requested one does not divide in_features (kernels/int4_linear.py:127-134)."""
        g = _group_for_from_float(linear.in_features, group_size)
        layer = cls(linear.in_features, linear.out_features, linear.bias is not None, g,
                    device or linear.weight.device)
        packed, scale = cls.quantize_weight(linear.weight, g)
        return layer.load_quantized(packed, scale, linear.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = _g.int4_linear(x, self.weight_packed, self.weight_scale, self.group_size)
        return y if self.bias is None else y + self.bias

    def extra_repr(self) -> str:
        return (f"in={self.in_features}, out={self.out_features}, int4 group={self.group_size}, "
                f"bias={self.bias is not None}")


def stacked_int4(layers: Sequence[Int4Linear]):
    """(packed, scale, group) of several Int4Linear layers of one input stacked
    along the output dimension, so one hn_int4_linear launch computes them all
    (the decoder's q/k/v projections)."""
    g = layers[0].group_size
    assert all(l.group_size == g and l.in_features == layers[0].in_features for l in layers), \
        "stacked_int4: layers differ in input size or group size"
    return (torch.cat([l.weight_packed for l in layers], 0),
            torch.cat([l.weight_scale for l in layers], 0), g)


@dataclass
class _ConversionReport:
    converted: List[str] = field(default_factory=list)
    skipped: Dict[str, str] = field(default_factory=dict)


def convert_model_to_int4(model: nn.Module, skip_layers: Optional[list] = None,
                          group_size: int = 128,
                          device: Optional[torch.device] = None) -> nn.Module:
    """Replace, in place, every nn.Linear whose qualified name contains none of
    ``skip_layers`` by an Int4Linear (kernels/int4_linear.py:174-236).  A layer
    with an odd in_features, or whose in_features no group of at least 32
    (halving from ``group_size``) divides, stays as it is.  Returns the model;
    ``model._int4_report`` lists what was converted and why layers were not."""
    patterns = list(skip_layers or [])
    report = _ConversionReport()
    targets = []
    for name, mod in model.named_modules():
        if not isinstance(mod, nn.Linear):
            continue
        if any(p in name for p in patterns):
            report.skipped[name] = "name matches skip_layers"
        elif mod.in_features % 2:
            report.skipped[name] = f"odd in_features={mod.in_features}"
        else:
            g = _group_for_convert(mod.in_features, group_size)
            if g is None:
                report.skipped[name] = f"no group >= {_MIN_GROUP} divides {mod.in_features}"
            else:
                targets.append((name, mod, g))
    for name, mod, g in targets:
        owner_name, _, attr = name.rpartition(".")
        owner = model.get_submodule(owner_name) if owner_name else model
        setattr(owner, attr, Int4Linear.from_float(mod, g, device))
        report.converted.append(name)
    model._int4_report = report
    print(f"convert_model_to_int4: {len(report.converted)} linear layers -> INT4, "
          f"{len(report.skipped)} kept")
    return model


def estimate_int4_memory(model: nn.Module, group_size: int = 128) -> dict:
    """Parameter bytes in fp16 against INT4 (kernels/int4_linear.py:239-269):
    every 2-D parameter as nibbles plus one fp16 scale per (row, group of
    ``group_size`` columns, rounded up), every other parameter kept in fp16.
    Megabytes (1e6 bytes): fp16_mb, int4_mb, savings_mb."""
    fp16 = int4 = 0
    for p in model.parameters():
        fp16 += 2 * p.numel()
        if p.dim() == 2:
            rows, cols = p.shape
            int4 += p.numel() // 2 + 2 * rows * (-(-cols // group_size))
        else:
            int4 += 2 * p.numel()
    return {"fp16_mb": fp16 / 1e6, "int4_mb": int4 / 1e6, "savings_mb": (fp16 - int4) / 1e6}

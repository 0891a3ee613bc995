"""Seeded synthetic experts for benchmarks and tests (no checkpoints offline).

Weights follow the reference tests' recipe, fp16 N(0, 0.02)
(tests/test_int4_loader.py:76-78), drawn on the GPU from a seeded torch
generator, then packed by the GPU packer (mode 0 = ExpertWeightPacker
arithmetic) straight into a GpuExpertSlot slab.  Mixtral naming: w1 = gate,
w3 = up, w2 = down (model/loader.py:160-164).
"""
from __future__ import annotations

import torch

from ..cache.packed_expert_store import GpuExpertSlot
from ..kernels.int4_gemm import quantize_int4


def expert_seed(layer: int, expert: int, base: int = 42) -> int:
    """Per-expert seed = base + layer*100 + expert (bench.py:191 in the reference)."""
    return base + layer * 100 + expert


def normal_f16(shape, seed: int, std: float = 0.02, device="cuda") -> torch.Tensor:
    g = torch.Generator(device=device).manual_seed(seed)
    return (torch.randn(*shape, generator=g, device=device, dtype=torch.float32) * std).to(
        torch.float16)


def make_expert_slot(seed: int, hidden_dim: int, intermediate_dim: int, group_size: int = 128,
                     device="cuda", slot_idx: int = 0) -> GpuExpertSlot:
    H, I = hidden_dim, intermediate_dim
    slot = GpuExpertSlot(slot_idx, H, I, group_size, torch.device(device))
    tensors = {}
    for j, (name, shape) in enumerate([("gate", (I, H)), ("up", (I, H)), ("down", (H, I))]):
        w = normal_f16(shape, seed * 3 + j, device=device)
        p, s = quantize_int4(w, group_size, mode=0)
        tensors[f"{name}_packed"], tensors[f"{name}_scales"] = p, s
        del w
    slot.load_from_tensors(tensors)
    return slot


def slot_to_cpu(slot: GpuExpertSlot):
    """(gp, gs, up, us, dp, ds) CPU copies, for the CPU oracle."""
    return tuple(getattr(slot, n).cpu() for n in ("gate_packed", "gate_scales", "up_packed",
                                                   "up_scales", "down_packed", "down_scales"))

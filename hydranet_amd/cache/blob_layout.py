"""Byte layout of one packed INT4 expert blob (the on-disk and in-HBM format).

Format fixed by the reference (cache/packed_expert_store.py:56-108,
written by preprocess/pack_glm4.py:102-119): six tensors back to back, no
padding, in the order

    gate_packed [I, H/2] u8 | gate_scales [I, H/g] f16 |
    up_packed   [I, H/2] u8 | up_scales   [I, H/g] f16 |
    down_packed [H, I/2] u8 | down_scales [H, I/g] f16

The field names (``<tensor>_offset`` / ``<tensor>_size``) and ``total_size``
match the reference so code written against it keeps working.
"""
from __future__ import annotations

from dataclasses import dataclass

TENSORS = ("gate_packed", "gate_scales", "up_packed", "up_scales", "down_packed", "down_scales")


@dataclass
class BlobLayout:
    gate_packed_offset: int = 0
    gate_packed_size: int = 0
    gate_scales_offset: int = 0
    gate_scales_size: int = 0
    up_packed_offset: int = 0
    up_packed_size: int = 0
    up_scales_offset: int = 0
    up_scales_size: int = 0
    down_packed_offset: int = 0
    down_packed_size: int = 0
    down_scales_offset: int = 0
    down_scales_size: int = 0

    @staticmethod
    def shapes(hidden_dim: int, intermediate_dim: int, group_size: int) -> dict:
        """name -> (shape, torch dtype name) for the six tensors."""
        H, I, g = hidden_dim, intermediate_dim, group_size
        return {
            "gate_packed": ((I, H // 2), "uint8"),
            "gate_scales": ((I, H // g), "float16"),
            "up_packed": ((I, H // 2), "uint8"),
            "up_scales": ((I, H // g), "float16"),
            "down_packed": ((H, I // 2), "uint8"),
            "down_scales": ((H, I // g), "float16"),
        }

    @classmethod
    def from_dims(cls, hidden_dim: int, intermediate_dim: int, group_size: int) -> "BlobLayout":
        layout = cls()
        cursor = 0
        for name, (shape, dtype) in cls.shapes(hidden_dim, intermediate_dim, group_size).items():
            nbytes = shape[0] * shape[1] * (1 if dtype == "uint8" else 2)
            setattr(layout, f"{name}_offset", cursor)
            setattr(layout, f"{name}_size", nbytes)
            cursor += nbytes
        return layout

    @property
    def total_size(self) -> int:
        return self.down_scales_offset + self.down_scales_size

    def spans(self):
        """[(name, offset, size)] in blob order."""
        return [(n, getattr(self, f"{n}_offset"), getattr(self, f"{n}_size")) for n in TENSORS]

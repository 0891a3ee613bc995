"""gfx950 kernels for the INT4 expert-MLP path.

Export surface of the reference's kernels/__init__.py:15-35 for this path.
Note the reference's name collision, kept here: the package-level
``expert_mlp_int4`` is ``expert_mlp.expert_mlp_int4`` (extra ``hidden_dim,
intermediate_dim`` arguments), not ``int4_expert_mlp.expert_mlp_int4``.
The INT8 exports (Int8Linear, ...) belong to attention/lm_head weights, which
are outside this path, and are not provided.
"""
from .expert_mlp import ExpertMLPTriton, expert_mlp_int4
from .int4_gemm import int4_linear, expert_mlp_int4_fused, fused_silu_mul
from .int4_linear import Int4Linear, convert_model_to_int4, estimate_int4_memory

__all__ = [
    "ExpertMLPTriton",
    "expert_mlp_int4",
    "int4_linear",
    "expert_mlp_int4_fused",
    "fused_silu_mul",
    "Int4Linear",
    "convert_model_to_int4",
    "estimate_int4_memory",
]

"""hydranet_amd — MI355X (gfx950) native INT4 expert-MLP hot path of HydraNet.

Layout:
  csrc/        hand-written HIP kernels + the C ABI (include/hn_int4.h)
  kernels/     drop-ins for the reference's kernels/int4_gemm.py,
               int4_expert_mlp.py, int4_linear.py, expert_mlp.py
  model/       routers and MoE-layer dispatch over the grouped kernels
  cache/       blob layout, GPU expert slots, pinned staging, packed store,
               per-layer INT4 slot cache
  preprocess/  INT4 packer and experts.bin / experts.idx writers
"""
__version__ = "0.1.0"

"""ctypes binding of libhn_int4.so (the C ABI declared in include/hn_int4.h).

torch is imported first on purpose: torch ships the HIP runtime
(libamdhip64.so.7), and loading it before this library makes the library bind
to the same runtime instance, so torch's streams and allocations are valid
here.  There is no fallback: if the library is missing or a call fails, the
caller gets a RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the CDLL load, see module doc)

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libhn_int4.so")

P = ctypes.c_void_p
L = ctypes.c_long
I = ctypes.c_int
F = ctypes.c_float

SIGNATURES: dict[str, list] = {
    "hn_int4_dequant": [P, L, P, L, P, L, L, L, L, P],
    "hn_int4_quantize": [P, L, I, I, P, L, P, L, L, L, L, P],
    "hn_skinny_workspace_bytes": [I, L, L, L, L],
    "hn_int4_linear": [P, L, P, L, P, L, P, L, L, L, L, L, P, L, P],
    "hn_int4_gate_up_silu": [P, L, P, P, P, P, L, L, P, L, L, L, L, L, P, L, P],
    "hn_expert_mlp_int4": [P, P, P, P, P, P, P, P, L, L, L, L, P, P, L, P],
    "hn_silu_mul": [P, L, P, L, P, L, L, L, P],
    "hn_silu_then_mul": [P, L, P, L, P, L, L, L, P],
    "hn_router_logits": [P, L, P, L, I, P, L, L, L, P],
    "hn_router_topk": [P, P, L, L, L, I, F, F, P, P, P],
    "hn_router_group_limit": [P, L, L, L, L, P, P],
    "hn_moe_permute": [P, L, L, L, P, P, P, P, P, P],
    "hn_moe_gather": [P, L, P, L, P, L, P, L, L, L, P],
    "hn_moe_unpermute": [P, L, P, P, P, L, L, P, L, P, L, L, P],
    "hn_add_rmsnorm": [P, L, P, L, P, L, P, P, L, L, L, F, P],
    "hn_add_rmsnorm_router": [P, L, P, L, P, L, P, P, L, L, L, F, P, L, L, P, P],
    "hn_attn_softmax": [P, L, P, L, L, L, L, F, P, L, P],
    "hn_attn_decode": [P, P, P, L, L, L, L, L, L, P, F, P, L, P],
    "hn_unpermute_add_rmsnorm": [P, L, L, P, P, P, L, L, P, L, P, L, P, P, L, L, F, P],
    "hn_moe_decode_layer_partials": [L, L, L, L, L],
    "hn_moe_experts_decode_split_check": [L, L, L, L, L, L],
    "hn_hbm_read_probe": [P, L, L, P, P],
    "hn_attn_decode_rope": [P, L, P, P, P, P, P, L, L, L, L, L, L, P, F, P, L, P],
    "hn_rope_append": [P, L, P, L, P, L, P, P, P, L, L, L, L, L, P, P, P, L, P],
    "hn_grouped_expert_mlp_int4": [P, P, P, P, P, L, L, L, L, L, L, P, P, P, L, P],
    "hn_set_decode_path": [I],
    "hn_gemm_workspace_bytes": [],
    "hn_grouped_expert_phase_int4": [I, P, P, P, P, P, L, L, L, L, L, P, P, P, L, P],
    "hn_moe_route": [P, L, P, L, I, P, P, L, L, L, L, I, F, F, P, P, P, P, P, P, P, P, P, P,
                     L, P],
    "hn_moe_experts_decode": [P, P, P, P, P, L, L, L, L, L, L, P, P, P, P, P, L, L, P, L, P, L,
                              P, L, P],
    "hn_grouped_decode_phase_int4": [I, P, P, P, P, P, L, L, L, L, L, L, P, P, L, P],
    "hn_moe_decode_layer_check": [L, L, L, L, L, L, I],
    "hn_moe_route_gate_up": [P, L, P, L, P, L, L, L, P, L, L, L, F, F, P, P, P, P, P, P, P, P,
                             P, P, P],
    "hn_moe_decode_layer": [P, L, P, L, P, L, L, L, P, L, L, L, F, F, P, P, P, P, P, P, P, P,
                            P, P, P, L, P, L, P],
    "hn_expert_mlp_int4_noalloc": [P, P, P, P, P, P, P, P, L, L, L, L, P],
    "hn_moe_route_experts_decode_check": [L, L, L, I, L, L, L],
    "hn_moe_route_experts_decode": [P, P, L, L, L, I, F, F, P, L, P, L, L, L, P, P, P, P, P, P,
                                    P, P, P, P, P, P, L, P, L, P, L, P],
}

# Sizes up to which hn_moe_route (one launch: logits, top-k, permutation,
# gather) applies; larger batches use the separate kernels.
ROUTE_MAX_LOGITS = 8192   # T * E
ROUTE_MAX_ASSIGN = 1024   # T * k

RESTYPES = {"hn_skinny_workspace_bytes": ctypes.c_long, "hn_gemm_workspace_bytes": ctypes.c_long,
            "hn_moe_decode_layer_partials": ctypes.c_long}

# Tokens per weight matrix up to which the decode (skinny / streaming) kernels
# run; above it the MFMA GEMM kernels do (kMaxRows in csrc/hn_gemv.hip).
DECODE_MAX_ROWS = 64

_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m hydranet_amd.build` "
                "(the INT4 path has no CPU fallback)")
        h = ctypes.CDLL(LIB_PATH)
        h.hn_last_error_string.restype = ctypes.c_char_p
        h.hn_abi_version.restype = ctypes.c_int
        for name, argtypes in SIGNATURES.items():
            fn = getattr(h, name)
            fn.argtypes = argtypes
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        _lib = h
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().hn_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{name} failed (rc={rc}): {msg}")


_DECODE_PATH = threading.local()


def set_decode_path(path: int) -> None:
    """Decode kernel family of the calling thread: 0 = the streaming kernels
    where they apply, 1 = split-K kernels only (A/B measurement and tests)."""
    call("hn_set_decode_path", path)
    _DECODE_PATH.value = path


def decode_path() -> int:
    return getattr(_DECODE_PATH, "value", 0)


_WORKSPACES: dict = {}
# Every workspace ever handed out, per device.  A captured HIP graph keeps the
# raw pointer of the workspace it was captured with, so a buffer superseded by
# a larger one must stay allocated (never return to the caching allocator)
# while such a graph may replay: the process keeps them all.
_RETIRED: dict = {}


def _device_key(dev: torch.device):
    if dev.type != "cuda":
        return (dev.type, 0)
    return (dev.type, dev.index if dev.index is not None else torch.cuda.current_device())


def workspace(nbytes: int, device) -> torch.Tensor:
    """Zero-filled scratch for the split-K counters and partials, cached per
    device and grown on demand.  The kernels leave the counters at zero, so
    the buffer is only filled once per allocation.  Calls that share a device
    run in stream order; concurrent calls on different streams would race.
    Growing keeps the old buffer allocated (see _RETIRED)."""
    dev = torch.device(device)
    key = _device_key(dev)
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        if buf is not None:
            _RETIRED.setdefault(key, []).append(buf)
        buf = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=dev)
        _WORKSPACES[key] = buf
    return buf


def skinny_workspace(kind: int, M: int, N: int, K: int, E: int, device) -> torch.Tensor:
    return workspace(lib().hn_skinny_workspace_bytes(kind, M, N, K, E), device)


def gemm_workspace(device) -> torch.Tensor:
    """Workspace of the prefill GEMM kernels' stream-K split (about 128 MiB)."""
    return workspace(lib().hn_gemm_workspace_bytes(), device)



def ptr(t) -> ctypes.c_void_p:
    if t is None:
        return ctypes.c_void_p(None)
    return ctypes.c_void_p(t.data_ptr())


def stream(device=None) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def require_gpu(*tensors) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(
                "hydranet_amd INT4 kernels run on the GPU only; got a tensor on "
                f"{t.device} (there is no CPU fallback)")


def aligned_rows(t: torch.Tensor) -> torch.Tensor:
    """Contiguous inner dim and a 16-byte aligned base, copying if needed."""
    if t.stride(-1) != 1 or t.data_ptr() % 16 != 0 or (t.dim() > 1 and
                                                         (t.stride(-2) * t.element_size()) % 16):
        t = t.contiguous()
        if t.data_ptr() % 16 != 0:
            t = t.clone()
    return t

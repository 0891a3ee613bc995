"""TEST INFRASTRUCTURE ONLY — CPU oracle for the INT4 expert-MLP hot path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker or the timed CPU
baseline.  The product (``hydranet_amd``) never imports it.

Two layers:

* ``liboracle.so`` (``hn_oracle.c``): plain-C restatements of the bit-level
  parts — packer, dequantiser, router top-k, permute/unpermute — each citing
  the reference line it follows.  Numpy arrays in and out.
* ``torch_ref`` : torch-CPU restatement of the reference's
  dequantise-then-matmul path (kernels/expert_mlp.py:292-330) and of the MoE
  layer dispatch (model/mixtral.py:283-368, model/glm4.py:365-473).

Pinning (what makes these trustworthy) lives in tests/test_oracle.py: golden
vectors written by the reference's own code (tests/golden/), the reference's
own test assertions, closed forms and brute force on tiny inputs.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None


def build() -> str:
    """Compile liboracle.so with the committed Makefile (gcc, plain C)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return os.path.join(_HERE, "liboracle.so")


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        _LIB = ctypes.CDLL(path)
    return _LIB


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


L = ctypes.c_long


def f16_bits(a: np.ndarray) -> np.ndarray:
    return _c(a, np.float16).view(np.uint16)


def quantize(w: np.ndarray, group: int, mode: int = 0):
    """Reference quantiser restated. w: fp16 or fp32 [N, K].
    mode 0 = ExpertWeightPacker.quantize_tensor, mode 1 = Int4Linear.quantize_weight.
    Returns (packed uint8 [N, K/2], scales fp16 [N, K/group])."""
    N, K = w.shape
    if w.dtype == np.float16:
        src, dtype = f16_bits(w), 0
    else:
        src, dtype = _c(w, np.float32), 1
    packed = np.empty((N, K // 2), np.uint8)
    scales = np.empty((N, K // group), np.uint16)
    lib().oracle_quantize(_p(src), ctypes.c_int(dtype), ctypes.c_int(mode), L(N), L(K), L(group),
                          _p(packed), _p(scales))
    return packed, scales.view(np.float16)


def dequant(packed: np.ndarray, scales: np.ndarray, group: int) -> np.ndarray:
    N = packed.shape[0]
    K = packed.shape[1] * 2
    out = np.empty((N, K), np.uint16)
    lib().oracle_dequant(_p(_c(packed, np.uint8)), _p(f16_bits(scales)), L(N), L(K), L(group),
                         _p(out))
    return out.view(np.float16)


def int4_linear(x: np.ndarray, packed: np.ndarray, scales: np.ndarray, group: int) -> np.ndarray:
    M, K = x.shape
    N = packed.shape[0]
    out = np.empty((M, N), np.uint16)
    lib().oracle_int4_linear(_p(f16_bits(x)), _p(_c(packed, np.uint8)), _p(f16_bits(scales)),
                             L(M), L(N), L(K), L(group), _p(out))
    return out.view(np.float16)


def router_logits(h: np.ndarray, w: np.ndarray) -> np.ndarray:
    T, H = h.shape
    E = w.shape[0]
    if w.dtype == np.float16:
        wsrc, wd = f16_bits(w), 0
    else:
        wsrc, wd = _c(w, np.float32), 1
    out = np.empty((T, E), np.float32)
    lib().oracle_router_logits(_p(f16_bits(h)), _p(wsrc), ctypes.c_int(wd), L(T), L(E), L(H),
                               _p(out))
    return out


def router_topk(logits: np.ndarray, k: int, mode: int, bias=None, eps: float = 1e-9,
                scaling: float = 1.0):
    T, E = logits.shape
    idx = np.empty((T, k), np.int32)
    w = np.empty((T, k), np.uint16)
    b = None if bias is None else _c(bias, np.float32)
    lib().oracle_router_topk(_p(_c(logits, np.float32)), None if b is None else _p(b), L(T), L(E),
                             L(k), ctypes.c_int(mode), ctypes.c_float(eps),
                             ctypes.c_float(scaling), _p(idx), _p(w))
    return idx, w.view(np.float16)


def router_group_limit(logits: np.ndarray, n_group: int, topk_group: int) -> np.ndarray:
    """Logits with -inf outside each token's topk_group best groups (max sigmoid)."""
    T, E = logits.shape
    out = np.empty((T, E), np.float32)
    lib().oracle_router_group_limit(_p(_c(logits, np.float32)), L(T), L(E), L(n_group),
                                    L(topk_group), _p(out))
    return out


def moe_permute(idx: np.ndarray, E: int):
    flat = _c(idx, np.int32).reshape(-1)
    n = flat.size
    offsets = np.empty(E + 1, np.int32)
    perm = np.full(max(n, 1), -1, np.int32)
    inv = np.empty(max(n, 1), np.int32)
    active = np.full(E, -1, np.int32)
    n_active = np.zeros(1, np.int32)
    lib().oracle_moe_permute(_p(flat), L(n), L(E), _p(offsets), _p(perm), _p(inv), _p(active),
                             _p(n_active))
    return offsets, perm[:n], inv[:n], active[: int(n_active[0])]


def moe_unpermute(y_perm: np.ndarray, inv: np.ndarray, idx: np.ndarray, w: np.ndarray,
                  shared=None) -> np.ndarray:
    T, k = idx.shape
    H = y_perm.shape[1]
    out = np.empty((T, H), np.uint16)
    sh = None if shared is None else f16_bits(shared)
    lib().oracle_moe_unpermute(_p(f16_bits(y_perm)), _p(_c(inv, np.int32)), _p(_c(idx, np.int32)),
                               _p(f16_bits(w)), L(T), L(k), None if sh is None else _p(sh), L(H),
                               _p(out))
    return out.view(np.float16)


def f32_to_f16_bits(a: np.ndarray) -> np.ndarray:
    src = _c(a, np.float32).reshape(-1)
    out = np.empty(src.size, np.uint16)
    lib().oracle_f32_to_f16(_p(src), _p(out), L(src.size))
    return out.reshape(np.shape(a))

"""Deterministic weights for the golden fixtures (test infrastructure).

The layer and store-format fixtures in this folder hold only small inputs and
outputs; their expert weights are regenerated from seeds by this module, in
make_golden.py (which hands them to the reference's code) and in the tests
(which hand them to the oracle and to this build).  So the values must be
the same on every machine: only integer operations and IEEE-exact float64
+, -, * (no log/sin/cos, whose last bits differ between math libraries).

``normal(seed, shape, std)`` is an Irwin-Hall approximation of N(0, std^2):
the sum of four 24-bit uniforms from a splitmix64 stream, centred and scaled
to unit variance, then rounded to float32.
"""
from __future__ import annotations

import hashlib

import numpy as np

_M = np.uint64(0xFFFFFFFFFFFFFFFF)


def _splitmix64(seed: int, n: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        i = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + i * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def normal(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """float32 array of the given shape, mean 0 and standard deviation std."""
    n = int(np.prod(shape))
    z = _splitmix64(seed, 4 * n).reshape(n, 4)
    u = (z >> np.uint64(40)).astype(np.int64)          # 24-bit uniforms
    s = u.sum(axis=1) - 2 * (1 << 24)                  # exact integer
    # the sum has variance 4 * 2^48 / 12, i.e. standard deviation 2^24 / sqrt(3)
    v = s.astype(np.float64) * (std * 1.7320508075688772 / float(1 << 24))
    return v.astype(np.float32).reshape(shape)


def normal_f16(seed: int, shape, std: float = 1.0) -> np.ndarray:
    return normal(seed, shape, std).astype(np.float16)


def sha256(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# seeds of the layer fixtures' weights
def expert_seeds(case_seed: int, e: int, layer: int = 0):
    """(gate, up, down) seeds of expert e of a layer."""
    b = (case_seed * 100 + layer) * 1000 + 10 * e
    return b, b + 1, b + 2


def expert_weights(case_seed: int, e: int, H: int, I: int, layer: int = 0) -> dict:
    """fp16 numpy {gate_proj [I, H], up_proj [I, H], down_proj [H, I]}, N(0, 0.02)
    like the reference tests' synthetic experts (tests/test_int4_loader.py:76-78)."""
    sg, su, sd = expert_seeds(case_seed, e, layer)
    return {"gate_proj": normal_f16(sg, (I, H), 0.02), "up_proj": normal_f16(su, (I, H), 0.02),
            "down_proj": normal_f16(sd, (H, I), 0.02)}

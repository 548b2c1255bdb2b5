"""Oracle restatement of the deterministic init spec (test infrastructure only).

Restates, in numpy, the counter-based generator the library implements
(hackathon_amd/csrc/host_init.hip) and the per-parameter ranges of the
reference's `randomize_` (check_cell_rewrite.py:187-210), written from that
function's rules rather than from the product's table:

  RGLRU.a U(0.1,0.9); Mamba2.a U(-16,-1); Mamba2.d U(0.5,1.5);
  RetNet.decay U(0.85,0.99); RetNet.angle U(0.01,0.2); learnable_skip
  U(0.9,1.1); norm weights U(0.9,1.1); biases and other norm params
  U(-0.05,0.05); everything else U(+-1/sqrt(shape[-1])).
"""

from __future__ import annotations

import math

import numpy as np

M64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15


def _mix64_int(z: int) -> int:
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def param_key(seed: int, name: str) -> int:
    h = 0xCBF29CE484222325
    for byte in name.encode():
        h ^= byte
        h = (h * 0x100000001B3) & M64
    return _mix64_int(h ^ _mix64_int(seed & M64))


def _mix64_np(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def uniform(seed: int, name: str, n: int, lo: float, hi: float) -> np.ndarray:
    key = np.uint64(param_key(seed, name))
    idx = np.arange(1, n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        bits = _mix64_np(key + idx * np.uint64(GOLDEN))
    u = (bits >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    lo32, hi32 = np.float32(lo), np.float32(hi)
    span = np.float32(hi32 - lo32)
    return (lo32 + (span * u).astype(np.float32)).astype(np.float32)


NORM_OWNERS = ("norm", "norm1", "norm2", "final_norm", "group_norm", "outnorm")


def range_for(name: str, shape) -> tuple[float, float]:
    """randomize_'s rule for one parameter (check_cell_rewrite.py:192-210)."""
    parts = name.split(".")
    leaf = parts[-1]
    owner = parts[-2] if len(parts) > 1 else ""
    grand = parts[-3] if len(parts) > 2 else ""
    if owner == "rglru" and leaf == "a":
        return 0.1, 0.9
    is_layer = owner == "layer"
    if is_layer and leaf == "a":
        return -16.0, -1.0          # Mamba2.a (the only `a` directly on a layer)
    if is_layer and leaf == "d":
        return 0.5, 1.5
    if is_layer and leaf == "decay":
        return 0.85, 0.99
    if is_layer and leaf == "angle":
        return 0.01, 0.2
    if leaf == "learnable_skip":
        return 0.9, 1.1
    if owner in NORM_OWNERS and leaf == "weight":
        return 0.9, 1.1
    if leaf == "bias" or owner in NORM_OWNERS:
        return -0.05, 0.05
    s = 1.0 / math.sqrt(shape[-1])
    return -s, s

"""Deterministic weights (the init spec in spec.py) generated on the host by
the library's counter-based filler, returned as CPU fp32 tensors keyed by the
reference's state_dict names."""

from __future__ import annotations

import ctypes
import os

import torch

from . import _lib
from .spec import ModelConfig, param_specs

_lib.register("hk_param_key", ctypes.c_uint64, [ctypes.c_uint64, ctypes.c_char_p])
_lib.register(
    "hk_fill_uniform_host",
    ctypes.c_int,
    [ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float, ctypes.c_float, ctypes.c_int],
)
_lib.register("hk_to_lp_host", ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int])

LP_FORMATS = {"bf16": 0, "fp16": 1}


def param_key(seed: int, name: str) -> int:
    return int(_lib.lib().hk_param_key(seed & (2**64 - 1), name.encode()))


def fill_uniform(t: torch.Tensor, seed: int, name: str, lo: float, hi: float) -> torch.Tensor:
    assert t.dtype == torch.float32 and t.device.type == "cpu" and t.is_contiguous()
    threads = min(32, os.cpu_count() or 1)
    st = _lib.lib().hk_fill_uniform_host(
        t.data_ptr(), t.numel(), param_key(seed, name), lo, hi, threads
    )
    _lib.check(st, "hk_fill_uniform_host")
    return t


def generate(cfg: ModelConfig, seed: int = 0) -> dict[str, torch.Tensor]:
    """All parameters of MultiTowerModel(cfg), initialised by the spec."""
    out = {}
    for p in param_specs(cfg):
        out[p.name] = fill_uniform(torch.empty(p.shape, dtype=torch.float32), seed, p.name, p.lo, p.hi)
    return out


def to_lp_bits(x: torch.Tensor, fmt: str) -> torch.Tensor:
    """16-bit patterns (int16 tensor) of fp32 values in CastLinear format
    `fmt` ("bf16" / "fp16"), by the library's host conversion
    (hk_to_lp_host), which rounds every non-NaN value as its kernels'
    device conversion does for weights, biases and activations."""
    x = x.detach().to(torch.float32).contiguous().cpu()
    out = torch.empty(x.shape, dtype=torch.int16)
    _lib.check(_lib.lib().hk_to_lp_host(x.data_ptr(), out.data_ptr(), x.numel(), LP_FORMATS[fmt]),
               "hk_to_lp_host")
    return out


def check_state_dict(cfg: ModelConfig, sd: dict, strict: bool = True) -> None:
    """Raise unless `sd` holds every parameter of MultiTowerModel(cfg) under
    the reference's names with the reference's shapes (and, with strict,
    nothing else), as torch's load_state_dict would."""
    want = {p.name: p.shape for p in param_specs(cfg)}
    missing = sorted(set(want) - set(sd))
    unexpected = sorted(set(sd) - set(want))
    if missing or (strict and unexpected):
        raise KeyError(f"state_dict mismatch: missing {missing[:5]} ({len(missing)}), "
                       f"unexpected {unexpected[:5]} ({len(unexpected)})")
    for k, shape in want.items():
        if tuple(sd[k].shape) != tuple(shape):
            raise ValueError(f"{k}: shape {tuple(sd[k].shape)}, expected {tuple(shape)}")


def load_checkpoint(path, cfg: ModelConfig) -> dict[str, torch.Tensor]:
    """A reference state_dict from a local file, read as the reference client
    reads its checkpoint (torch.load with weights_only=True,
    example_model.py:296-302; the download itself needs the network), checked
    against cfg and converted to CPU fp32."""
    sd = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(sd, dict):
        raise ValueError(f"{path}: expected a state_dict, found {type(sd).__name__}")
    check_state_dict(cfg, sd)
    return {k: v.detach().to(torch.float32).contiguous() for k, v in sd.items()}

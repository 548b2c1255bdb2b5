"""Model configuration, parameter inventory and the deterministic init spec.

`ModelConfig` mirrors model/inference_model.py:21-27; the defaults are the
dimensions the reference client hard-codes (example_model.py:283-289). The
per-layer constants are create_layer's (model/inference_model.py:30-52):
Mamba2 head 64 / bc 128, sLSTM heads = heads // 2, mLSTM heads = heads.

`param_specs` lists every floating parameter and buffer under the exact
state_dict name the reference model registers, with the uniform range that
check_cell_rewrite.py:187-210 (`randomize_`) assigns it. Values come from the
counter-based generator in the library (hk_fill_uniform_host), so weights are
a pure function of (seed, name, element index).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

TOWER_TYPES = ("xlstm", "mamba2", "retnet", "hawk")  # model/inference_model.py:107-112

# example_model.py:106 - linears that CastLinear never converts.
FP32_LINEAR_NAMES = ("dt_proj", "igate_proj", "fgate_proj", "output_proj")


@dataclass(frozen=True)
class ModelConfig:
    hidden_size: int = 2048
    proj_size: int = 4096
    tower_depth: int = 12
    num_heads: int = 8
    num_features: int = 79
    mamba_head_size: int = 64
    mamba_bc_size: int = 128

    @property
    def inner(self) -> int:
        return 2 * self.hidden_size

    @property
    def slstm_heads(self) -> int:
        return self.num_heads // 2

    @property
    def mamba_heads(self) -> int:
        return self.inner // self.mamba_head_size

    @property
    def retnet_head(self) -> int:
        return self.hidden_size // self.num_heads

    @property
    def mlstm_head(self) -> int:
        return self.inner // self.num_heads


DEFAULT = ModelConfig()
SMALL = ModelConfig(hidden_size=64, proj_size=128, tower_depth=2, num_heads=4, num_features=7)


@dataclass(frozen=True)
class ParamSpec:
    name: str
    shape: tuple
    lo: float
    hi: float

    @property
    def numel(self) -> int:
        return math.prod(self.shape)


def _lin(shape):
    s = 1.0 / math.sqrt(shape[-1])
    return (-s, s)


NORM = (0.9, 1.1)
BIAS = (-0.05, 0.05)


def _layer_params(cfg: ModelConfig, ltype: str):
    H, I = cfg.hidden_size, cfg.inner
    out = []

    def p(name, shape, rng=None):
        lo, hi = rng if rng is not None else _lin(shape)
        out.append((name, tuple(shape), lo, hi))

    if ltype == "xlstm":
        nh_s, bs = cfg.slstm_heads, H // cfg.slstm_heads
        p("slstm.norm.weight", (H,), NORM)
        p("slstm.conv1d.conv.weight", (H, 1, 4))
        p("slstm.conv1d.conv.bias", (H,), BIAS)
        for g in "ifzo":
            p(f"slstm.{g}gate_input.weight", (nh_s, bs, bs))
        for g in "ifzo":
            p(f"slstm.{g}gate_state.weight", (nh_s, bs, bs))
            p(f"slstm.{g}gate_state.bias", (H,), BIAS)
        p("slstm.group_norm.weight", (H,), NORM)
        p("slstm.group_norm.bias", (H,), BIAS)
        p("mlstm.norm.weight", (H,), NORM)
        p("mlstm.x_proj.weight", (I, H))
        p("mlstm.gate_proj.weight", (I, H))
        for g in "qkv":
            p(f"mlstm.{g}_proj.weight", (I // 4, 4, 4))
        p("mlstm.conv1d.conv.weight", (I, 1, 4))
        p("mlstm.conv1d.conv.bias", (I,), BIAS)
        for g in ("igate", "fgate"):
            p(f"mlstm.mlstm_cell.{g}_proj.weight", (cfg.num_heads, 3 * I))
            p(f"mlstm.mlstm_cell.{g}_proj.bias", (cfg.num_heads,), BIAS)
        p("mlstm.mlstm_cell.outnorm.weight", (I,), NORM)
        p("mlstm.mlstm_cell.outnorm.bias", (I,), BIAS)
        p("mlstm.proj_down.weight", (H, I))
        p("mlstm.learnable_skip", (I,), (0.9, 1.1))
        p("final_norm.weight", (H,), NORM)
    elif ltype == "mamba2":
        nhm, bc = cfg.mamba_heads, cfg.mamba_bc_size
        p("a", (nhm,), (-16.0, -1.0))
        p("d", (nhm,), (0.5, 1.5))
        p("input_proj.weight", (I, H))
        p("z_proj.weight", (I, H))
        p("b_proj.weight", (bc, H))
        p("c_proj.weight", (bc, H))
        p("dt_proj.weight", (nhm, H))
        p("dt_proj.bias", (nhm,), BIAS)
        p("input_conv.conv.weight", (I, 1, 4))
        p("input_conv.conv.bias", (I,), BIAS)
        p("b_conv.conv.weight", (bc, 1, 4))
        p("b_conv.conv.bias", (bc,), BIAS)
        p("c_conv.conv.weight", (bc, 1, 4))
        p("c_conv.conv.bias", (bc,), BIAS)
        p("norm.weight", (I,), NORM)
        p("out_proj.weight", (H, I))
    elif ltype == "retnet":
        for g in "qkvg":
            p(f"{g}_proj.weight", (H, H))
        p("out_proj.weight", (H, H))
        p("decay", (cfg.num_heads,), (0.85, 0.99))
        p("angle", (cfg.retnet_head,), (0.01, 0.2))
    elif ltype == "hawk":
        bs = H // 4
        p("gate_proj.weight", (H, H))
        p("recurrent_proj.weight", (H, H))
        p("conv.conv.weight", (H, 1, 4))
        p("conv.conv.bias", (H,), BIAS)
        p("rglru.input_gate.weight", (4, bs, bs))
        p("rglru.recurrence_gate.weight", (4, bs, bs))
        p("rglru.a", (H,), (0.1, 0.9))
        p("out_proj.weight", (H, H))
    else:
        raise ValueError(ltype)
    return out


def param_specs(cfg: ModelConfig) -> list[ParamSpec]:
    """Every floating parameter/buffer of MultiTowerModel(cfg), reference names."""
    H, P, F = cfg.hidden_size, cfg.proj_size, cfg.num_features
    specs = []
    for t, ltype in enumerate(TOWER_TYPES):
        pre = f"towers.{t}."
        specs.append(ParamSpec(pre + "input_up.weight", (P, F), *_lin((P, F))))
        specs.append(ParamSpec(pre + "input_up.bias", (P,), *BIAS))
        specs.append(ParamSpec(pre + "input_down.weight", (H, P), *_lin((H, P))))
        specs.append(ParamSpec(pre + "input_down.bias", (H,), *BIAS))
        for b in range(cfg.tower_depth):
            bp = f"{pre}blocks.{b}."
            specs.append(ParamSpec(bp + "norm1.weight", (H,), *NORM))
            for name, shape, lo, hi in _layer_params(cfg, ltype):
                specs.append(ParamSpec(bp + "layer." + name, shape, lo, hi))
            specs.append(ParamSpec(bp + "norm2.weight", (H,), *NORM))
            specs.append(ParamSpec(bp + "mlp.fc1.weight", (P, H), *_lin((P, H))))
            specs.append(ParamSpec(bp + "mlp.fc1.bias", (P,), *BIAS))
            specs.append(ParamSpec(bp + "mlp.fc2.weight", (H, P), *_lin((H, P))))
            specs.append(ParamSpec(bp + "mlp.fc2.bias", (H,), *BIAS))
    specs.append(ParamSpec("output_proj.weight", (1, H), *_lin((1, H))))
    specs.append(ParamSpec("output_proj.bias", (1,), *BIAS))
    return specs


def is_cast_linear(name: str) -> bool:
    """True for nn.Linear weights/biases that CastLinear converts
    (example_model.py:109-148): every Linear except FP32_LINEAR_NAMES.
    BlockLinear, conv, norm parameters and buffers are never converted."""
    parts = name.split(".")
    if parts[-1] not in ("weight", "bias") or len(parts) < 2:
        return False
    owner = parts[-2]
    linear_owners = {
        "input_up", "input_down", "fc1", "fc2", "input_proj", "z_proj", "b_proj", "c_proj",
        "dt_proj", "out_proj", "q_proj", "k_proj", "v_proj", "g_proj", "gate_proj",
        "recurrent_proj", "x_proj", "proj_down", "igate_proj", "fgate_proj", "output_proj",
    }
    if owner not in linear_owners or owner in FP32_LINEAR_NAMES:
        return False
    # q/k/v_proj inside the mLSTM block are BlockLinear, not nn.Linear.
    if owner in ("q_proj", "k_proj", "v_proj") and ".mlstm." in f".{name}":
        return False
    return True

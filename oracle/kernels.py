"""Oracle for the three fused state steps (test infrastructure only).

Restates the reference's torch twins and their write-back contract:
- `_write_back`            model/kernels.py:124-137
- `mlstm_step_reference`   model/kernels.py:143-151
- `retnet_step_reference`  model/kernels.py:154-160
- `mamba2_step_reference`  model/kernels.py:163-171

Works in whatever dtype its inputs have (fp32 for parity, fp64 for the
brute-force checks in tests/test_oracle_kernels.py).
"""

from __future__ import annotations

import torch


def write_back(state, new, out, mask, batch):
    """Masked in-place write of `new`; zeros in `out`'s idle rows (kernels.py:124-137)."""
    if mask is None:
        state.copy_(new)
        return out
    state.copy_(torch.where(mask.view(batch, 1, 1, 1), new, state))
    return torch.where(mask.view(batch, 1, 1), out, out.new_zeros(()))


def mlstm_step(cell, q, k, v, i_gate, f_gate, mask):
    """cell <- f*cell + (i*k) outer v; return sum_h q*cell_new (kernels.py:143-151)."""
    batch = cell.shape[0]
    cell_new = (
        f_gate[:, :, None, None] * cell
        + i_gate[:, :, None, None] * k[:, :, :, None] * v[:, :, None, :]
    )
    numerator = (q[:, :, :, None] * cell_new).sum(dim=2)
    return write_back(cell, cell_new, numerator, mask, batch)


def retnet_step(state, k_rope, v, q_scaled, decay, mask):
    """state <- decay*state + k outer v; return sum_h q_scaled*state_new (kernels.py:154-160)."""
    batch = state.shape[0]
    outer = k_rope[:, :, :, None] * v[:, :, None, :]
    state_new = state * decay[None, :, None, None] + outer
    out = (q_scaled[:, :, :, None] * state_new).sum(dim=2)
    return write_back(state, state_new, out, mask, batch)


def mamba2_step(ssm, x, b, c, dt, decay, mask):
    """ssm <- decay*ssm + (dt*b) outer x; return sum_c c*ssm_new (kernels.py:163-171)."""
    batch = ssm.shape[0]
    ssm_new = (
        decay[:, :, None, None] * ssm
        + dt[:, :, None, None] * b[:, None, None, :] * x[:, :, :, None]
    )
    y = (c[:, None, None, :] * ssm_new).sum(dim=-1)
    return write_back(ssm, ssm_new, y, mask, batch)
